/* A C caller of libllmk_sampler.so, built against include/llmk_sampler.h
 * with -std=c99 -Wall -Wextra -Werror -pedantic: the argument checks every
 * entry point makes before it touches a device, their return codes and
 * llmk_last_error() messages.  Needs no GPU.  Prints "ok N" and returns 0
 * when every check holds; otherwise names the first failed check. */
#include <stdio.h>
#include <string.h>

#include "llmk_sampler.h"

static int n_checks = 0;

#define CHECK(cond)                                                       \
  do {                                                                    \
    ++n_checks;                                                           \
    if (!(cond)) {                                                        \
      printf("FAILED line %d: %s (last error: \"%s\")\n", __LINE__, #cond, \
             llmk_last_error());                                          \
      return 1;                                                           \
    }                                                                     \
  } while (0)

static int has(const char* needle) { return strstr(llmk_last_error(), needle) != NULL; }

int main(void) {
  llmk_sampler* s = (llmk_sampler*)0x1; /* must be cleared on failure */
  llmk_sample_batch_args a;
  uint32_t st = 0;
  memset(&a, 0, sizeof(a));

  /* llmk_sampler_create */
  CHECK(llmk_sampler_create(NULL, 0, 1, 1) == LLMK_ERR_INVALID_ARGUMENT);
  CHECK(has("out is NULL"));
  CHECK(llmk_sampler_create(&s, 0, 0, 1000) == LLMK_ERR_INVALID_ARGUMENT);
  CHECK(s == NULL);
  CHECK(has("max_batch"));
  CHECK(llmk_sampler_create(&s, 0, 4, 0) == LLMK_ERR_INVALID_ARGUMENT);
  CHECK(llmk_sampler_create(&s, 0, 4, (1u << 20) + 1) == LLMK_ERR_CAPACITY);
  CHECK(s == NULL);

  /* llmk_sample_batch, llmk_sample_batch_static */
  CHECK(llmk_sample_batch(NULL, &a, NULL) == LLMK_ERR_INVALID_ARGUMENT);
  CHECK(has("NULL"));
  CHECK(llmk_sample_batch_static(NULL, NULL, NULL) == LLMK_ERR_INVALID_ARGUMENT);
  CHECK(has("args is NULL"));
  a.batch = 257;
  a.vocab = 1000;
  CHECK(llmk_sample_batch_static(&a, NULL, NULL) == LLMK_ERR_CAPACITY);
  CHECK(has("batch <= 256"));
  a.batch = 1;
  a.vocab = (1u << 18) + 1;
  CHECK(llmk_sample_batch_static(&a, &st, NULL) == LLMK_ERR_CAPACITY);

  /* the mask forms and logit bias */
  {
    float* lg = (float*)0x1000;
    const int32_t* k = (const int32_t*)0x2000;
    const float* p = (const float*)0x3000;
    const uint32_t* u = (const uint32_t*)0x4000;
    CHECK(llmk_apply_top_k(NULL, lg, 1, 8, 8, k, NULL) == LLMK_ERR_INVALID_ARGUMENT);
    CHECK(has("sampler is NULL"));
    CHECK(llmk_apply_top_p(NULL, lg, 1, 8, 8, p, NULL) == LLMK_ERR_INVALID_ARGUMENT);
    CHECK(llmk_apply_logit_bias(NULL, lg, 1, 8, 8, u, u, p, NULL) == LLMK_ERR_INVALID_ARGUMENT);
  }

  /* histories, verification, status */
  CHECK(llmk_history_append(NULL, 1, NULL, NULL, NULL, 8, NULL, NULL) ==
        LLMK_ERR_INVALID_ARGUMENT);
  CHECK(llmk_history_count_append(NULL, 1, NULL, NULL, NULL, NULL, 8, NULL, NULL) ==
        LLMK_ERR_INVALID_ARGUMENT);
  CHECK(llmk_verify_batch(NULL, 1, 8, NULL, NULL, 4, NULL, NULL, NULL, 8, NULL, NULL, NULL, NULL,
                          NULL) == LLMK_ERR_INVALID_ARGUMENT);
  CHECK(llmk_sampler_status(NULL, NULL, &st) == LLMK_ERR_INVALID_ARGUMENT);
  llmk_sampler_destroy(NULL); /* a no-op */

  /* the constants and the layout a binding mirrors */
  CHECK(LLMK_INVALID_TOKEN == 0xffffffffu);
  CHECK(sizeof(llmk_sample_batch_args) == 192);
  CHECK(sizeof(void*) == 8);

  printf("ok %d\n", n_checks);
  return 0;
}
