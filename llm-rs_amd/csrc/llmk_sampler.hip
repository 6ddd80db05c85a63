// llmk_sampler.hip — MI355X (gfx950) batched token sampling for llm-rs.
//
// Replaces the host loop llm-scheduler/src/scheduler.rs:138-145, which calls
// llm-core/src/sampler.rs:25-125 (sample_logits) once per row, with one
// stream-ordered call that samples the whole batch on the GPU.
//
// Kernels
//   stream_kernel   one workgroup per (row, vocabulary segment).  Reads the
//                   logits of its segment once from HBM (128-bit / 64-bit
//                   non-temporal loads), applies the penalties (from an LDS
//                   bitmap + hash of the row's history), the allow-mask, and
//                   per 1024-token tile computes the tile max and
//                   sum 2^((l - max) log2(e)/T) (the softmax normaliser's
//                   partial) — or the tile argmax for greedy rows — and
//                   collects top-candidates above a rising threshold kept
//                   in an LDS histogram over the logits' order-preserving
//                   keys.  The last workgroup of a row to finish (arrival
//                   counter) runs `finalize`: merges the tile partials into
//                   the normaliser S, computes exact probabilities of the
//                   candidates, sorts them by (p desc, idx asc), proves that
//                   no non-candidate can precede the ones it uses, and runs
//                   min-p / top-k / top-p / the draw exactly as sampler.rs.
//   slow_kernel     rows the fast path cannot prove exact (top-k = 0 with a
//                   large nucleus, candidate overflow, fully masked rows):
//                   exact probabilities of the whole row, stable LSD radix
//                   sort in global memory, the same sequential semantics.
//
// Numerics are fixed (llmk_numerics.h); the CPU mirror oracle restates them.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdio>
#include <cstring>
#include <string>

#include "llmk_numerics.h"
#include "llmk_sampler.h"

namespace llmk {

constexpr uint32_t TILE = 1024;      // canonical vocabulary tile
constexpr int WAVE = 64;
constexpr int NW = 8;                // waves per stream workgroup
constexpr int NT = NW * WAVE;        // 512 threads
constexpr uint32_t NBINS = 4096;     // fine histogram bins: key >> 20
constexpr uint32_t BIN_SHIFT = 20;
constexpr uint32_t CBIN_SHIFT = 26;  // coarse bins: key >> 26 (64 bins)
constexpr uint32_t HASH_SLOTS = 8192;
constexpr uint32_t HASH_MAX_PROBE = 1024;
constexpr uint32_t CAND_CAP = 8192;  // candidate entries per workgroup
constexpr uint32_t SORT_CAP = 4096;  // candidates sorted in finalize
constexpr uint32_t KMAX = 2048;      // largest top-k served by the fast path
constexpr uint32_t KCAND_NOK = 512;  // candidate target when top-k is off
constexpr uint32_t MAX_TILES = 1024; // max_vocab <= 2^20
constexpr uint32_t MAX_WGS = 4096;   // candidate-buffer pool entries
constexpr int SLOW_NT = 1024;        // slow-path workgroup
constexpr uint32_t SLOW_WGS = 64;    // concurrent slow rows
constexpr uint32_t EMPTY = 0xffffffffu;
constexpr float NEG_INF = -__builtin_huge_valf();

enum : uint32_t { MODE_INVALID = 0, MODE_GREEDY = 1, MODE_SAMPLE = 2 };
enum : uint32_t { FLAG_OVERFLOW = 1u, FLAG_HIST_OVERFLOW = 2u };

struct Args {
  const void* logits;
  int32_t dtype;
  uint32_t B, V;
  uint64_t stride;
  const float *T, *top_p, *min_p, *rp, *pp, *fp;
  const int32_t* top_k;
  const uint32_t *hoff, *htok, *mask;
  uint32_t mask_words;
  const float* u;
  uint32_t *out_tok, *out_ids, *out_cnt;
  float* out_probs;
  uint32_t out_cap;
  uint32_t G, tps, ntiles;
  uint32_t xcd_map;  // 1: segments of a row share an XCD
};

struct Ws {
  uint32_t* row_arrive;  // [max_batch]
  float2* tile_part;     // [max_batch][MAX_TILES]
  uint4* seg_meta;       // [pool]: count, beta, flags, -
  uint2* cand;           // [pool][CAND_CAP]: value bits, index
  uint32_t* row_flags;   // [max_batch]: 1 = needs slow path
  float4* row_stats;     // [max_batch]: S, m, L, -
  uint64_t* slow_keys;   // [SLOW_WGS][3][max_vocab]
  float* slow_p;         // [SLOW_WGS][max_vocab]
  uint32_t* slow_idx;    // [SLOW_WGS][max_vocab]
  uint32_t* status;      // [1]
  uint32_t max_vocab;
};

struct RowP {
  float T, top_p, min_p, rp, pp, fp;
  int32_t K;
  uint32_t mode;
  uint32_t Kc;  // candidate target; 0 = fast path impossible
};

__device__ __forceinline__ bool finitef(float x) { return __builtin_isfinite(x); }

__device__ RowP row_params(const Args& a, uint32_t b) {
  RowP r;
  r.T = a.T ? a.T[b] : 1.0f;
  r.top_p = a.top_p ? a.top_p[b] : 1.0f;
  r.min_p = a.min_p ? a.min_p[b] : 0.0f;
  r.rp = a.rp ? a.rp[b] : 1.0f;
  r.pp = a.pp ? a.pp[b] : 0.0f;
  r.fp = a.fp ? a.fp[b] : 0.0f;
  r.K = a.top_k ? a.top_k[b] : 0;
  const bool bad = !finitef(r.T) || r.K < 0 || !finitef(r.top_p) ||
                   !finitef(r.min_p) || !(r.min_p >= 0.0f) || !finitef(r.rp) ||
                   !finitef(r.pp) || !finitef(r.fp);
  r.mode = bad ? MODE_INVALID : (r.T <= 1e-5f ? MODE_GREEDY : MODE_SAMPLE);
  const bool topk_on = r.K > 0 && (uint32_t)r.K < a.V;
  r.Kc = topk_on ? ((uint32_t)r.K <= KMAX ? (uint32_t)r.K : 0u) : KCAND_NOK;
  return r;
}

// ---------------------------------------------------------------------------
// Wave helpers (wave64)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t x) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_xor(x, o);
    x = y < x ? y : x;
  }
  return x;
}
// Balanced-tree sum over lanes 0..63 (lane pairs (2i,2i+1), then pairs of
// pairs, ...): every lane ends with the same value.
__device__ __forceinline__ float wave_tree_sum(float x) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) x = x + __shfl_xor(x, o);
  return x;
}
__device__ __forceinline__ uint32_t wave_incl_prefix(uint32_t x, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  return x;
}

// ---------------------------------------------------------------------------
// History: LDS bitmap over a vocabulary range + hash of counts
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t hslot(uint32_t t) {
  return (t * 2654435761u) >> (32 - 13);  // HASH_SLOTS = 2^13
}

__device__ bool hash_insert(uint32_t* hk, uint32_t* hc, uint32_t t) {
  uint32_t s = hslot(t);
  for (uint32_t n = 0; n < HASH_MAX_PROBE; ++n) {
    const uint32_t old = atomicCAS(&hk[s], EMPTY, t);
    if (old == EMPTY || old == t) {
      atomicAdd(&hc[s], 1u);
      return true;
    }
    s = (s + 1) & (HASH_SLOTS - 1);
  }
  return false;
}

__device__ uint32_t hash_count(const uint32_t* hk, const uint32_t* hc,
                               uint32_t t) {
  uint32_t s = hslot(t);
  for (uint32_t n = 0; n < HASH_MAX_PROBE; ++n) {
    const uint32_t k = hk[s];
    if (k == t) return hc[s];
    if (k == EMPTY) return 0;
    s = (s + 1) & (HASH_SLOTS - 1);
  }
  return 0;
}

// Fill bitmap[(t-lo)>>5] and the hash for history tokens t in [lo, hi).
template <int NTH>
__device__ void build_history(const Args& a, const RowP& P, uint32_t b,
                              uint32_t lo, uint32_t hi, uint32_t nwords,
                              uint32_t* bitmap, uint32_t* hk, uint32_t* hc,
                              uint32_t* flags) {
  const uint32_t tid = threadIdx.x;
  for (uint32_t i = tid; i < nwords; i += NTH) bitmap[i] = 0;
  const bool need_cnt = P.fp != 0.0f;
  if (need_cnt)
    for (uint32_t i = tid; i < HASH_SLOTS; i += NTH) {
      hk[i] = EMPTY;
      hc[i] = 0;
    }
  __syncthreads();
  const bool need_pen = P.rp != 1.0f || P.pp != 0.0f || P.fp != 0.0f;
  if (need_pen && a.hoff && a.htok) {
    const uint32_t h0 = a.hoff[b], h1 = a.hoff[b + 1];
    for (uint32_t i = h0 + tid; i < h1; i += NTH) {
      const uint32_t t = a.htok[i];
      if (t >= lo && t < hi) {
        atomicOr(&bitmap[(t - lo) >> 5], 1u << (t & 31));
        if (need_cnt && !hash_insert(hk, hc, t)) atomicOr(flags, FLAG_HIST_OVERFLOW);
      }
    }
  }
  __syncthreads();
}

// Penalties on one logit of a history token (sampler.rs:139-143, then the
// presence/frequency formula of llm-tests/tests/mlc_parity.rs:1083).
__device__ __forceinline__ float penalize(float x, const RowP& P,
                                          uint32_t count) {
  if (P.rp != 1.0f) x = (x > 0.0f) ? x / P.rp : x * P.rp;
  if (P.pp != 0.0f || P.fp != 0.0f) {
    const float cf = (float)count * P.fp;
    x = x - (P.pp + cf);
  }
  return x;
}

// ---------------------------------------------------------------------------
// Candidate-threshold histogram
// ---------------------------------------------------------------------------
// Largest fine bin beta such that at least Kc counted elements have bin >=
// beta (0 if fewer than Kc are counted).  Counts are lower bounds of the true
// counts, so the result never exceeds the bin of the true Kc-th largest.
__device__ uint32_t compute_beta(const uint32_t* hc, const uint32_t* hf,
                                 uint32_t Kc, int lane) {
  const uint32_t c = hc[63 - lane];
  const uint32_t incl = wave_incl_prefix(c, lane);
  const uint64_t m = __ballot(incl >= Kc);
  if (m == 0) return 0;
  const int l = __ffsll((unsigned long long)m) - 1;
  const uint32_t cb = 63u - (uint32_t)l;
  const uint32_t before = __shfl(incl - c, l);
  const uint32_t need = Kc - before;
  const uint32_t f = hf[cb * 64 + 63 - lane];
  const uint32_t fincl = wave_incl_prefix(f, lane);
  const uint64_t m2 = __ballot(fincl >= need);
  if (m2 == 0) return 0;
  const int l2 = __ffsll((unsigned long long)m2) - 1;
  return cb * 64u + 63u - (uint32_t)l2;
}

// ---------------------------------------------------------------------------
// Geometry helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ void wg_to_row_seg(const Args& a, uint32_t i,
                                              uint32_t& b, uint32_t& g) {
  if (a.xcd_map) {
    const uint32_t x = i & 7u, j = i >> 3;
    b = x + 8u * (j / a.G);
    g = j % a.G;
  } else {
    b = i / a.G;
    g = i % a.G;
  }
}
__device__ __forceinline__ uint32_t row_seg_to_wg(const Args& a, uint32_t b,
                                                  uint32_t g) {
  if (a.xcd_map) return 8u * (a.G * (b >> 3) + g) + (b & 7u);
  return b * a.G + g;
}

// ---------------------------------------------------------------------------
// Tile loads
// ---------------------------------------------------------------------------
typedef float f4v __attribute__((ext_vector_type(4)));
typedef uint32_t u2v __attribute__((ext_vector_type(2)));

struct Raw {
  uint32_t d[16];   // fp32 bits (or 8 dwords of bf16 pairs)
  uint32_t mw[4];   // allow-mask words for the lane's 4 groups
};

// Lane `lane` owns tile offsets 256r + 4*lane + q (r, q in 0..3).
template <int DT>
__device__ __forceinline__ void load_tile(const Args& a, const void* row,
                                          const uint32_t* mrow, uint32_t t,
                                          int lane, Raw& raw) {
  const uint32_t tb = t * TILE;
  if (tb + TILE <= a.V) {
    if (DT == LLMK_F32) {
      const f4v* p = (const f4v*)((const float*)row + tb) + lane;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const f4v x = __builtin_nontemporal_load(p + 64 * r);
        raw.d[4 * r + 0] = __float_as_uint(x.x);
        raw.d[4 * r + 1] = __float_as_uint(x.y);
        raw.d[4 * r + 2] = __float_as_uint(x.z);
        raw.d[4 * r + 3] = __float_as_uint(x.w);
      }
    } else {
      const u2v* p = (const u2v*)((const uint16_t*)row + tb) + lane;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const u2v x = __builtin_nontemporal_load(p + 64 * r);
        raw.d[2 * r + 0] = x.x;
        raw.d[2 * r + 1] = x.y;
      }
    }
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t e = tb + 256u * r + 4u * lane + q;
        uint32_t bits = 0xff800000u;  // -inf beyond the vocabulary
        if (e < a.V) {
          if (DT == LLMK_F32) bits = ((const uint32_t*)row)[e];
          else bits = (uint32_t)((const uint16_t*)row)[e] << 16;
        }
        if (DT == LLMK_F32) raw.d[4 * r + q] = bits;
        else {
          // repack into the bf16 pair layout used by the full-tile path
          const uint32_t h = bits >> 16;
          const int w = 2 * r + (q >> 1);
          if ((q & 1) == 0) raw.d[w] = h;
          else raw.d[w] |= h << 16;
        }
      }
  }
  if (mrow) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t wi = (tb >> 5) + 8u * r + ((uint32_t)lane >> 3);
      raw.mw[r] = (wi < a.mask_words) ? mrow[wi] : 0u;
    }
  }
}

template <int DT>
__device__ __forceinline__ void unpack(const Raw& raw, float v[16]) {
  if (DT == LLMK_F32) {
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = __uint_as_float(raw.d[j]);
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      v[4 * r + 0] = __uint_as_float(raw.d[2 * r] << 16);
      v[4 * r + 1] = __uint_as_float(raw.d[2 * r] & 0xffff0000u);
      v[4 * r + 2] = __uint_as_float(raw.d[2 * r + 1] << 16);
      v[4 * r + 3] = __uint_as_float(raw.d[2 * r + 1] & 0xffff0000u);
    }
  }
}

// ---------------------------------------------------------------------------
// Shared-memory layout of the stream kernel
// ---------------------------------------------------------------------------
enum : uint32_t { M_BETA = 0, M_CCOUNT = 1, M_FLAGS = 2, M_LAST = 3, M_NMISC = 16 };

struct StreamLds {
  uint32_t* bitmap;  // tps*32
  uint32_t* hk;      // HASH_SLOTS
  uint32_t* hc;      // HASH_SLOTS
  uint32_t* hf;      // NBINS
  uint32_t* hcoarse; // 64
  uint32_t* misc;    // M_NMISC
};

__host__ __device__ inline size_t stream_lds_words(uint32_t tps) {
  return (size_t)tps * 32 + 2 * HASH_SLOTS + NBINS + 64 + M_NMISC;
}
// finalize: tile arrays 2*MAX_TILES floats, keys SORT_CAP u64, p/idx SORT_CAP
__host__ __device__ inline size_t finalize_lds_words() {
  return 2 * MAX_TILES + 2 * SORT_CAP + 2 * SORT_CAP + 64;
}

// ---------------------------------------------------------------------------
// Finalize one row (one workgroup of NT threads)
// ---------------------------------------------------------------------------
__device__ float block_max(float x, float* red) {
  x = wave_max(x);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wv] = x;
  __syncthreads();
  float r = red[0];
  for (int i = 1; i < NT / WAVE; ++i) r = fmaxf(r, red[i]);
  __syncthreads();
  return r;
}
__device__ uint32_t block_min_u32(uint32_t x, uint32_t* red) {
  x = wave_min_u32(x);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wv] = x;
  __syncthreads();
  uint32_t r = red[0];
  for (int i = 1; i < NT / WAVE; ++i) r = red[i] < r ? red[i] : r;
  __syncthreads();
  return r;
}

// p of a (penalised, masked) logit v given the row's temperature, x_max = m
// and normaliser S: exactly sampler.rs:53-70 with exp_m.
__device__ __forceinline__ float prob_of(float v, float T, float m, float S) {
  const float x = (T != 1.0f) ? v / T : v;
  const float e = (x == NEG_INF) ? 0.0f : exp_m(x - m);
  return (S > 0.0f) ? e / S : e;
}

__device__ __forceinline__ uint64_t pkey(float p, uint32_t idx) {
  return ((uint64_t)(~__float_as_uint(p)) << 32) | idx;
}

// Sequential semantics of sampler.rs:77-124 (+ min-p) over a list sorted by
// (p desc, idx asc) of which the first E entries are known exactly and the
// list has `len` entries in total.  Executed by all threads of the block;
// thread 0 does the order-dependent sums, all threads the divisions.
// Returns false if the semantics need an entry beyond E.
template <typename PAcc, typename IAcc, int NTH>
__device__ bool run_semantics(const RowP& P, float u, uint32_t E,
                              uint32_t full_len, PAcc pget, IAcc iget,
                              uint32_t* sh, uint32_t& tok_out,
                              uint32_t& len_out) {
  // sh[0]=ok, sh[1]=len, sh[2]=trunc, sh[3]=sum bits, sh[4]=tok
  const uint32_t tid = threadIdx.x;
  if (tid == 0) {
    sh[0] = 1;
    sh[1] = full_len;
    sh[2] = (E < full_len) ? 1u : 0u;
  }
  __syncthreads();
  // ---- min-p (extension): keep p >= min_p * p_max, renormalise if cut
  if (P.min_p > 0.0f) {
    if (tid == 0) {
      uint32_t len = sh[1], ok = 1, cut = len;
      float s = 0.0f;
      bool do_norm = false;
      if (E == 0) ok = 0;
      else {
        const float thr = P.min_p * pget(0);
        uint32_t j = 0;
        bool found = false;
        for (; j < E && j < len; ++j)
          if (pget(j) < thr) {
            found = true;
            break;
          }
        if (found) cut = j;
        else if (sh[2] && E < len) ok = 0;
        if (ok && cut < len) {
          for (uint32_t i = 0; i < cut; ++i) s += pget(i);
          do_norm = true;
          sh[1] = cut;
          sh[2] = 0;
        }
      }
      sh[0] = ok;
      sh[3] = do_norm ? __float_as_uint(s) : 0u;
      sh[5] = do_norm ? 1u : 0u;
    }
    __syncthreads();
    if (!sh[0]) return false;
    if (sh[5]) {
      const float s = __uint_as_float(sh[3]);
      if (s > 0.0f)
        for (uint32_t i = tid; i < sh[1]; i += NTH) pget.set(i, pget(i) / s);
    }
    __syncthreads();
  }
  // ---- top-k, sampler.rs:80-89
  if (P.K > 0 && (uint32_t)P.K < sh[1]) {
    if (tid == 0) {
      const uint32_t K = (uint32_t)P.K;
      if (K > E) sh[0] = 0;
      else {
        float s = 0.0f;
        for (uint32_t i = 0; i < K; ++i) s += pget(i);
        sh[1] = K;
        sh[2] = 0;
        sh[3] = __float_as_uint(s);
      }
    }
    __syncthreads();
    if (!sh[0]) return false;
    const float s = __uint_as_float(sh[3]);
    if (s > 0.0f)
      for (uint32_t i = tid; i < sh[1]; i += NTH) pget.set(i, pget(i) / s);
    __syncthreads();
  }
  // ---- top-p, sampler.rs:92-110
  if (P.top_p < 1.0f) {
    if (tid == 0) {
      const uint32_t len = sh[1];
      float cum = 0.0f;
      uint32_t cut = len, j = 0;
      uint32_t ok = 1;
      for (; j < len; ++j) {
        if (j >= E) {
          ok = 0;
          break;
        }
        cum += pget(j);
        if (cum >= P.top_p) {
          cut = j + 1;
          break;
        }
      }
      sh[0] = ok;
      if (ok) {
        // the renormalisation sum over the kept prefix is the same
        // sequential sum as the cumulative at the cut
        sh[1] = cut;
        sh[2] = 0;
        sh[3] = __float_as_uint(cum);
      }
    }
    __syncthreads();
    if (!sh[0]) return false;
    const float s = __uint_as_float(sh[3]);
    if (s > 0.0f)
      for (uint32_t i = tid; i < sh[1]; i += NTH) pget.set(i, pget(i) / s);
    __syncthreads();
  }
  // ---- draw, sampler.rs:113-124
  if (tid == 0) {
    const uint32_t len = sh[1];
    uint32_t ok = 1, tok = 0;
    if (len > 0) {
      if (len - 1 < E) tok = iget(len - 1);
      else tok = EMPTY;  // fallback index unknown unless reached below
    }
    float cum = 0.0f;
    bool hit = false;
    for (uint32_t j = 0; j < len; ++j) {
      if (j >= E) {
        ok = 0;
        break;
      }
      cum += pget(j);
      if (u <= cum) {
        tok = iget(j);
        hit = true;
        break;
      }
    }
    if (!hit && tok == EMPTY) ok = 0;
    sh[0] = ok;
    sh[4] = tok;
  }
  __syncthreads();
  if (!sh[0]) return false;
  tok_out = sh[4];
  len_out = sh[1];
  return true;
}

struct LdsP {
  float* p;
  __device__ float operator()(uint32_t i) const { return p[i]; }
  __device__ void set(uint32_t i, float x) const { p[i] = x; }
};
struct LdsI {
  const uint32_t* p;
  __device__ uint32_t operator()(uint32_t i) const { return p[i]; }
};

__device__ void write_outputs(const Args& a, uint32_t b, uint32_t tok,
                              uint32_t len, const float* pp,
                              const uint32_t* pidx, uint32_t E, int nth) {
  const uint32_t tid = threadIdx.x;
  if (tid == 0) {
    a.out_tok[b] = tok;
    if (a.out_cnt) a.out_cnt[b] = len;
  }
  if (a.out_cap) {
    const uint32_t n = len < a.out_cap ? len : a.out_cap;
    for (uint32_t j = tid; j < n; j += nth) {
      if (a.out_ids) a.out_ids[(uint64_t)b * a.out_cap + j] = pidx[j];
      if (a.out_probs) a.out_probs[(uint64_t)b * a.out_cap + j] = pp[j];
    }
  }
}

__device__ void finalize_row(const Args& a, const Ws& w, uint32_t b,
                             const RowP& P, uint32_t* smem) {
  const uint32_t tid = threadIdx.x;
  float* tl = (float*)smem;                         // MAX_TILES
  float* ts = tl + MAX_TILES;                       // MAX_TILES
  uint64_t* keys = (uint64_t*)(smem + 2 * MAX_TILES);  // SORT_CAP
  float* pp = (float*)(keys + SORT_CAP);            // SORT_CAP
  uint32_t* pidx = (uint32_t*)(pp + SORT_CAP);      // SORT_CAP
  uint32_t* fm = pidx + SORT_CAP;                   // 64 words
  const uint32_t nt = a.ntiles;
  const float2* part = w.tile_part + (uint64_t)b * MAX_TILES;
  for (uint32_t c = tid; c < nt; c += NT) {
    const float2 q = part[c];
    tl[c] = q.x;
    ts[c] = q.y;
  }
  __syncthreads();

  if (P.mode == MODE_GREEDY) {
    // sampler.rs:40-50: the first index holding the maximum.
    float m = NEG_INF;
    for (uint32_t c = tid; c < nt; c += NT) m = fmaxf(m, tl[c]);
    m = block_max(m, (float*)fm);
    uint32_t bi = EMPTY;
    for (uint32_t c = tid; c < nt; c += NT)
      if (tl[c] == m) {
        const uint32_t ci = __float_as_uint(ts[c]);
        bi = ci < bi ? ci : bi;
      }
    bi = block_min_u32(bi, fm + 16);
    if (bi == EMPTY) bi = 0;
    if (tid == 0) {
      a.out_tok[b] = bi;
      if (a.out_cnt) a.out_cnt[b] = 1;
      if (a.out_cap) {
        if (a.out_ids) a.out_ids[(uint64_t)b * a.out_cap] = bi;
        if (a.out_probs) a.out_probs[(uint64_t)b * a.out_cap] = 1.0f;
      }
    }
    return;
  }

  // ---- normaliser S
  float L = NEG_INF;
  for (uint32_t c = tid; c < nt; c += NT) L = fmaxf(L, tl[c]);
  L = block_max(L, (float*)fm);
  const float c2 = LOG2E_F / P.T;
  uint32_t ntp = 1;
  while (ntp < nt) ntp <<= 1;
  for (uint32_t c = tid; c < ntp; c += NT) {
    float x = 0.0f;
    if (c < nt && L != NEG_INF) x = ts[c] * exp2_f((tl[c] - L) * c2);
    ts[c] = x;
  }
  __syncthreads();
  for (uint32_t len = ntp; len > 1; len >>= 1) {
    float x[MAX_TILES / NT];
    uint32_t k = 0;
    for (uint32_t i = tid; i < len / 2; i += NT) x[k++] = ts[2 * i] + ts[2 * i + 1];
    __syncthreads();
    k = 0;
    for (uint32_t i = tid; i < len / 2; i += NT) ts[i] = x[k++];
    __syncthreads();
  }
  const float S = (L != NEG_INF) ? ts[0] : 0.0f;
  const float m = (P.T != 1.0f) ? L / P.T : L;
  if (tid == 0) w.row_stats[b] = make_float4(S, m, L, 0.0f);

  // ---- candidates
  if (tid == 0) {
    uint32_t lam = 0, flags = 0, total = 0;
    for (uint32_t g = 0; g < a.G; ++g) {
      const uint4 sm = w.seg_meta[row_seg_to_wg(a, b, g)];
      const uint32_t lk = sm.y << BIN_SHIFT;
      lam = lk > lam ? lk : lam;
      flags |= sm.z;
      total += sm.x;
    }
    fm[32] = lam;
    fm[33] = flags;
    fm[34] = 0;  // gathered count
    fm[35] = (L == NEG_INF || P.Kc == 0 || (flags & FLAG_OVERFLOW)) ? 1u : 0u;
  }
  __syncthreads();
  bool slow = fm[35] != 0;
  const uint32_t lam = fm[32];
  if (!slow) {
    for (uint32_t g = 0; g < a.G; ++g) {
      const uint32_t wg = row_seg_to_wg(a, b, g);
      const uint32_t cnt = min(w.seg_meta[wg].x, CAND_CAP);
      const uint2* cb = w.cand + (uint64_t)wg * CAND_CAP;
      for (uint32_t i = tid; i < cnt; i += NT) {
        const uint2 e = cb[i];
        if (fkey(__uint_as_float(e.x)) >= lam) {
          const uint32_t pos = atomicAdd(&fm[34], 1u);
          if (pos < SORT_CAP)
            keys[pos] = pkey(prob_of(__uint_as_float(e.x), P.T, m, S), e.y);
        }
      }
    }
    __syncthreads();
    if (fm[34] > SORT_CAP) slow = true;
  }
  if (!slow) {
    const uint32_t n = fm[34];
    uint32_t npad = 1;
    while (npad < n) npad <<= 1;
    for (uint32_t i = n + tid; i < npad; i += NT) keys[i] = ~0ull;
    __syncthreads();
    for (uint32_t k = 2; k <= npad; k <<= 1)
      for (uint32_t j = k >> 1; j > 0; j >>= 1) {
        for (uint32_t i = tid; i < npad; i += NT) {
          const uint32_t ixj = i ^ j;
          if (ixj > i) {
            const uint64_t x = keys[i], y = keys[ixj];
            const bool up = (i & k) == 0;
            if ((x > y) == up) {
              keys[i] = y;
              keys[ixj] = x;
            }
          }
        }
        __syncthreads();
      }
    // P_lim: largest probability any non-candidate can have.
    if (tid == 0) {
      float plim = 0.0f;
      if (lam > 0x007fffffu) plim = prob_of(funkey(lam - 1), P.T, m, S);
      fm[36] = __float_as_uint(plim);
      fm[37] = n;  // E
    }
    __syncthreads();
    const float plim = __uint_as_float(fm[36]);
    for (uint32_t i = tid; i < n; i += NT) {
      const float p = __uint_as_float(~(uint32_t)(keys[i] >> 32));
      pp[i] = p;
      pidx[i] = (uint32_t)keys[i];
      if (!(p > plim)) atomicMin(&fm[37], i);
    }
    __syncthreads();
    const uint32_t E = fm[37];
    const float u = a.u[b];
    uint32_t tok = 0, len = 0;
    const bool ok = run_semantics<LdsP, LdsI, NT>(P, u, E, a.V, LdsP{pp},
                                                  LdsI{pidx}, fm + 40, tok, len);
    if (ok && a.out_cap && len > E && a.out_cap > E) slow = true;
    if (!ok) slow = true;
    if (!slow) {
      write_outputs(a, b, tok, len, pp, pidx, E, NT);
      return;
    }
  }
  if (tid == 0) w.row_flags[b] = 1u;
}

// ---------------------------------------------------------------------------
// Stream kernel
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(NT) void stream_kernel(Args a, Ws w) {
  extern __shared__ __align__(16) uint32_t smem[];
  const uint32_t tid = threadIdx.x;
  const int lane = (int)(tid & 63), wv = (int)(tid >> 6);
  uint32_t b, g;
  wg_to_row_seg(a, blockIdx.x, b, g);
  const RowP P = row_params(a, b);
  if (P.mode == MODE_INVALID) {
    if (g == 0 && tid == 0) {
      a.out_tok[b] = LLMK_INVALID_TOKEN;
      if (a.out_cnt) a.out_cnt[b] = 0;
      atomicOr(w.status, LLMK_STATUS_INVALID_PARAMS);
    }
    return;
  }
  const uint32_t t0 = g * a.tps;
  const uint32_t t1 = min(t0 + a.tps, a.ntiles);
  StreamLds S;
  S.bitmap = smem;
  S.hk = S.bitmap + (size_t)a.tps * 32;
  S.hc = S.hk + HASH_SLOTS;
  S.hf = S.hc + HASH_SLOTS;
  S.hcoarse = S.hf + NBINS;
  S.misc = S.hcoarse + 64;
  const bool collect = P.mode == MODE_SAMPLE && P.Kc > 0;
  if (collect) {
    for (uint32_t i = tid; i < NBINS; i += NT) S.hf[i] = 0;
    if (tid < 64) S.hcoarse[tid] = 0;
  }
  if (tid < M_NMISC) S.misc[tid] = 0;
  const uint32_t lo = t0 * TILE;
  const uint32_t hi = min(a.V, t1 * TILE);
  build_history<NT>(a, P, b, lo, hi, (t1 - t0) * 32, S.bitmap, S.hk, S.hc,
                    &S.misc[M_FLAGS]);
  const bool need_pen = P.rp != 1.0f || P.pp != 0.0f || P.fp != 0.0f;
  const bool need_cnt = P.fp != 0.0f;
  const void* row = (const char*)a.logits +
                    (uint64_t)b * a.stride * (DT == LLMK_F32 ? 4u : 2u);
  const uint32_t* mrow = a.mask ? a.mask + (uint64_t)b * a.mask_words : nullptr;
  float2* part = w.tile_part + (uint64_t)b * MAX_TILES;
  uint2* cbuf = w.cand + (uint64_t)blockIdx.x * CAND_CAP;
  const float c2 = LOG2E_F / P.T;
  const float NINF = NEG_INF;

  auto process = [&](const Raw& raw, uint32_t t) {
    float v[16];
    unpack<DT>(raw, v);
    const uint32_t tb = t * TILE;
    if (need_pen) {
      uint32_t nib[4];
      bool anyf = false;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t o = (t - t0) * TILE + 256u * r + 4u * lane;
        nib[r] = (S.bitmap[o >> 5] >> (o & 31)) & 0xfu;
        anyf |= nib[r] != 0;
      }
      if (anyf) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if ((nib[r] >> q) & 1u) {
              const uint32_t tok = tb + 256u * r + 4u * lane + q;
              const uint32_t cnt = need_cnt ? hash_count(S.hk, S.hc, tok) : 1u;
              v[4 * r + q] = penalize(v[4 * r + q], P, cnt);
            }
      }
    }
    if (mrow) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t nib = (raw.mw[r] >> ((4u * lane) & 31u)) & 0xfu;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (!((nib >> q) & 1u)) v[4 * r + q] = NINF;
      }
    }
    float lm = NINF;
#pragma unroll
    for (int j = 0; j < 16; ++j) lm = v[j] > lm ? v[j] : lm;
    lm = wave_max(lm);
    if (P.mode == MODE_GREEDY) {
      uint32_t bi = EMPTY;
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float x = v[4 * r + q];
          const uint32_t e = tb + 256u * r + 4u * lane + q;
          const bool hit = (x == lm) || (lm == NINF && !(x > NINF));
          if (hit && e < a.V && e < bi) bi = e;
        }
      bi = wave_min_u32(bi);
      if (lane == 0) part[t] = make_float2(lm, __uint_as_float(bi));
      return;
    }
    float s = 0.0f;
    if (lm != NINF) {
      float sr[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float e0 = exp2_f((v[4 * r + 0] - lm) * c2);
        const float e1 = exp2_f((v[4 * r + 1] - lm) * c2);
        const float e2 = exp2_f((v[4 * r + 2] - lm) * c2);
        const float e3 = exp2_f((v[4 * r + 3] - lm) * c2);
        sr[r] = wave_tree_sum((e0 + e1) + (e2 + e3));
      }
      s = (sr[0] + sr[1]) + (sr[2] + sr[3]);
    }
    if (lane == 0) part[t] = make_float2(lm, s);
    if (!collect) return;
    // ---- candidates above the rising histogram threshold
    uint32_t beta = __atomic_load_n(&S.misc[M_BETA], __ATOMIC_RELAXED);
    uint32_t k[16];
    bool pass[16];
    bool anyp = false;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      k[j] = fkey(v[j]);
      pass[j] = (v[j] > NINF) && ((k[j] >> BIN_SHIFT) >= beta);
      anyp |= pass[j];
    }
    if (!__any(anyp)) return;
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (pass[j]) {
        atomicAdd(&S.hf[k[j] >> BIN_SHIFT], 1u);
        atomicAdd(&S.hcoarse[k[j] >> CBIN_SHIFT], 1u);
      }
    const uint32_t nb = compute_beta(S.hcoarse, S.hf, P.Kc, lane);
    if (nb > beta) {
      if (lane == 0) atomicMax(&S.misc[M_BETA], nb);
      beta = nb;
    }
    uint32_t cnt = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      pass[j] = pass[j] && ((k[j] >> BIN_SHIFT) >= beta);
      cnt += pass[j] ? 1u : 0u;
    }
    const uint32_t incl = wave_incl_prefix(cnt, lane);
    const uint32_t tot = __shfl(incl, 63);
    if (tot == 0) return;
    uint32_t base = 0;
    if (lane == 0) base = atomicAdd(&S.misc[M_CCOUNT], tot);
    base = __shfl(base, 0);
    if (base + tot > CAND_CAP) {
      if (lane == 0) atomicOr(&S.misc[M_FLAGS], FLAG_OVERFLOW);
      return;
    }
    uint32_t pos = base + incl - cnt;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (pass[4 * r + q])
          cbuf[pos++] = make_uint2(__float_as_uint(v[4 * r + q]),
                                   tb + 256u * r + 4u * lane + q);
  };

  Raw ra, rb;
  uint32_t t = t0 + (uint32_t)wv;
  if (t < t1) load_tile<DT>(a, row, mrow, t, lane, ra);
  for (;;) {
    if (t >= t1) break;
    if (t + NW < t1) load_tile<DT>(a, row, mrow, t + NW, lane, rb);
    process(ra, t);
    t += NW;
    if (t >= t1) break;
    if (t + NW < t1) load_tile<DT>(a, row, mrow, t + NW, lane, ra);
    process(rb, t);
    t += NW;
  }

  // ---- publish the segment, find the row's last workgroup
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const uint32_t fl = S.misc[M_FLAGS];
    w.seg_meta[blockIdx.x] = make_uint4(S.misc[M_CCOUNT], S.misc[M_BETA], fl, 0u);
    if (fl & FLAG_HIST_OVERFLOW) atomicOr(w.status, LLMK_STATUS_HISTORY_OVERFLOW);
    uint32_t last = 1;
    if (a.G > 1) {
      __threadfence();
      const uint32_t old = atomicAdd(&w.row_arrive[b], 1u);
      last = (old == a.G - 1) ? 1u : 0u;
    }
    S.misc[M_LAST] = last;
  }
  __syncthreads();
  if (!S.misc[M_LAST]) return;
  __threadfence();
  if (tid == 0 && a.G > 1) w.row_arrive[b] = 0;
  finalize_row(a, w, b, P, smem);
}

// ---------------------------------------------------------------------------
// Slow path: exact probabilities of the whole row, stable radix sort
// ---------------------------------------------------------------------------
struct GlobP {
  float* p;
  __device__ float operator()(uint32_t i) const { return p[i]; }
  __device__ void set(uint32_t i, float x) const { p[i] = x; }
};
struct GlobI {
  const uint32_t* p;
  __device__ uint32_t operator()(uint32_t i) const { return p[i]; }
};

// Block-wide exclusive scan of one flag per thread (SLOW_NT threads).
__device__ uint32_t block_excl_scan_flag(bool f, uint32_t* red,
                                         uint32_t& total) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const uint64_t m = __ballot(f);
  const uint32_t below = __popcll(m & ((1ull << lane) - 1ull));
  if (lane == 0) red[wv] = __popcll(m);
  __syncthreads();
  uint32_t off = 0, tot = 0;
  for (int i = 0; i < SLOW_NT / WAVE; ++i) {
    const uint32_t c = red[i];
    if (i < wv) off += c;
    tot += c;
  }
  __syncthreads();
  total = tot;
  return off + below;
}

template <int DT>
__global__ __launch_bounds__(SLOW_NT) void slow_kernel(Args a, Ws w) {
  extern __shared__ __align__(16) uint32_t smem[];
  const uint32_t tid = threadIdx.x;
  const int lane = (int)(tid & 63), wv = (int)(tid >> 6);
  const uint32_t V = a.V;
  uint32_t* bitmap = smem;                       // ceil(V/32)
  const uint32_t nwords = (V + 31) / 32;
  uint32_t* hk = bitmap + ((nwords + 3) & ~3u);  // HASH_SLOTS
  uint32_t* hc = hk + HASH_SLOTS;                // HASH_SLOTS
  uint32_t* red = hc + HASH_SLOTS;               // 64
  uint32_t* sh = red + 64;                       // 64
  uint32_t* digit_off = sh + 64;                 // 256
  uint32_t* wcnt = digit_off + 256;              // 16*256
  uint32_t* ttot = wcnt + 16 * 256;              // 256
  for (uint32_t b = blockIdx.x; b < a.B; b += gridDim.x) {
    if (__atomic_load_n(&w.row_flags[b], __ATOMIC_RELAXED) == 0) continue;
    const RowP P = row_params(a, b);
    if (tid < 64) sh[tid] = 0;
    build_history<SLOW_NT>(a, P, b, 0, V, nwords, bitmap, hk, hc, &sh[10]);
    const bool need_pen = P.rp != 1.0f || P.pp != 0.0f || P.fp != 0.0f;
    const bool need_cnt = P.fp != 0.0f;
    const float4 st = w.row_stats[b];
    const float S = st.x, m = st.y;
    const uint64_t slot = blockIdx.x;
    uint64_t* kA = w.slow_keys + slot * 3 * (uint64_t)w.max_vocab;
    uint64_t* kB = kA + w.max_vocab;
    uint32_t* zl = (uint32_t*)(kB + w.max_vocab);  // zero-probability indices
    float* plist = w.slow_p + slot * (uint64_t)w.max_vocab;
    uint32_t* ilist = w.slow_idx + slot * (uint64_t)w.max_vocab;
    const void* row = (const char*)a.logits +
                      (uint64_t)b * a.stride * (DT == LLMK_F32 ? 4u : 2u);
    const uint32_t* mrow = a.mask ? a.mask + (uint64_t)b * a.mask_words : nullptr;
    // pass 1: exact p of every element, stable split into p>0 / p==0 lists
    uint32_t npos = 0, nzero = 0;
    for (uint32_t base = 0; base < V; base += SLOW_NT) {
      const uint32_t e = base + tid;
      float p = 0.0f;
      bool valid = e < V;
      if (valid) {
        float x;
        if (DT == LLMK_F32) x = ((const float*)row)[e];
        else x = __uint_as_float((uint32_t)((const uint16_t*)row)[e] << 16);
        if (need_pen && ((bitmap[e >> 5] >> (e & 31)) & 1u))
          x = penalize(x, P, need_cnt ? hash_count(hk, hc, e) : 1u);
        if (mrow && !((mrow[e >> 5] >> (e & 31)) & 1u)) x = NEG_INF;
        if (!(x > NEG_INF)) x = NEG_INF;  // NaN acts as -inf
        p = prob_of(x, P.T, m, S);
      }
      uint32_t tot;
      const uint32_t pos = block_excl_scan_flag(valid && p > 0.0f, red, tot);
      if (valid && p > 0.0f) kA[npos + pos] = pkey(p, e);
      npos += tot;
      const uint32_t zpos = block_excl_scan_flag(valid && !(p > 0.0f), red, tot);
      if (valid && !(p > 0.0f)) zl[nzero + zpos] = e;
      nzero += tot;
    }
    // stable LSD radix sort of kA[0..npos) on bits 32..63, 4 passes of 8 bits
    uint64_t* src = kA;
    uint64_t* dst = kB;
    for (int pass = 0; pass < 4; ++pass) {
      const int sh_bits = 32 + 8 * pass;
      if (tid < 256) digit_off[tid] = 0;
      __syncthreads();
      for (uint32_t i = tid; i < npos; i += SLOW_NT)
        atomicAdd(&digit_off[(uint32_t)(src[i] >> sh_bits) & 255u], 1u);
      __syncthreads();
      if (tid == 0) {
        uint32_t acc = 0;
        for (int d = 0; d < 256; ++d) {
          const uint32_t c = digit_off[d];
          digit_off[d] = acc;
          acc += c;
        }
      }
      __syncthreads();
      for (uint32_t base = 0; base < npos; base += SLOW_NT) {
        const uint32_t i = base + tid;
        const bool valid = i < npos;
        const uint64_t key = valid ? src[i] : 0ull;
        const uint32_t d = (uint32_t)(key >> sh_bits) & 255u;
        uint64_t peers = __ballot(valid);
#pragma unroll
        for (int bit = 0; bit < 8; ++bit) {
          const uint64_t bb = __ballot(((d >> bit) & 1u) != 0);
          peers &= ((d >> bit) & 1u) ? bb : ~bb;
        }
        const uint32_t rank = __popcll(peers & ((1ull << lane) - 1ull));
        for (uint32_t j = tid; j < 16 * 256; j += SLOW_NT) wcnt[j] = 0;
        __syncthreads();
        if (valid && rank == 0) wcnt[wv * 256 + d] = __popcll(peers);
        __syncthreads();
        if (tid < 256) {
          uint32_t acc = 0;
          for (int q = 0; q < SLOW_NT / WAVE; ++q) {
            const uint32_t c = wcnt[q * 256 + tid];
            wcnt[q * 256 + tid] = acc;
            acc += c;
          }
          ttot[tid] = acc;
        }
        __syncthreads();
        if (valid) dst[digit_off[d] + wcnt[wv * 256 + d] + rank] = key;
        __syncthreads();
        if (tid < 256) digit_off[tid] += ttot[tid];
        __syncthreads();
      }
      uint64_t* tmp = src;
      src = dst;
      dst = tmp;
    }
    // unpack into p / idx lists (sorted positives, then zeros by index)
    for (uint32_t i = tid; i < npos; i += SLOW_NT) {
      const uint64_t k = src[i];
      plist[i] = __uint_as_float(~(uint32_t)(k >> 32));
      ilist[i] = (uint32_t)k;
    }
    for (uint32_t i = tid; i < nzero; i += SLOW_NT) {
      plist[npos + i] = 0.0f;
      ilist[npos + i] = zl[i];
    }
    __threadfence_block();
    __syncthreads();
    uint32_t tok = 0, len = 0;
    const float u = a.u[b];
    run_semantics<GlobP, GlobI, SLOW_NT>(P, u, V, V, GlobP{plist},
                                         GlobI{ilist}, sh + 20, tok, len);
    __threadfence_block();
    __syncthreads();
    write_outputs(a, b, tok, len, plist, ilist, V, SLOW_NT);
    if (tid == 0) w.row_flags[b] = 0;
    __syncthreads();
  }
}

size_t slow_lds_bytes(uint32_t V) {
  const uint32_t nwords = (V + 31) / 32;
  return 4 * ((size_t)((nwords + 3) & ~3u) + 2 * HASH_SLOTS + 64 + 64 + 256 +
              16 * 256 + 256);
}

}  // namespace llmk

// ===========================================================================
// C ABI
// ===========================================================================
using namespace llmk;

struct llmk_sampler {
  int device;
  uint32_t max_batch, max_vocab;
  Ws ws;
  void* mem;
  size_t mem_bytes;
};

static thread_local std::string g_last_error;

static int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

extern "C" const char* llmk_last_error(void) { return g_last_error.c_str(); }

#define HIPCHK(expr)                                                        \
  do {                                                                      \
    hipError_t e_ = (expr);                                                 \
    if (e_ != hipSuccess)                                                   \
      return fail(LLMK_ERR_HIP, std::string(#expr " failed: ") +            \
                                    hipGetErrorString(e_));                 \
  } while (0)

static size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

extern "C" int llmk_sampler_create(llmk_sampler** out, int device,
                                   uint32_t max_batch, uint32_t max_vocab) {
  if (!out) return fail(LLMK_ERR_INVALID_ARGUMENT, "out is NULL");
  *out = nullptr;
  if (max_batch == 0 || max_vocab == 0)
    return fail(LLMK_ERR_INVALID_ARGUMENT, "max_batch and max_vocab must be > 0");
  if (max_vocab > MAX_TILES * TILE)
    return fail(LLMK_ERR_CAPACITY, "max_vocab above 2^20");
  HIPCHK(hipSetDevice(device));
  // Dynamic LDS above 64 KiB must be allowed explicitly.
  HIPCHK(hipFuncSetAttribute((const void*)stream_kernel<LLMK_F32>,
                             hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
  HIPCHK(hipFuncSetAttribute((const void*)stream_kernel<LLMK_BF16>,
                             hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
  HIPCHK(hipFuncSetAttribute((const void*)slow_kernel<LLMK_F32>,
                             hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
  HIPCHK(hipFuncSetAttribute((const void*)slow_kernel<LLMK_BF16>,
                             hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
  const uint32_t pool = max_batch > MAX_WGS ? max_batch : MAX_WGS;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off = align_up(off + bytes, 256);
    return o;
  };
  const size_t o_arrive = take(4ull * max_batch);
  const size_t o_part = take(8ull * max_batch * MAX_TILES);
  const size_t o_meta = take(16ull * pool);
  const size_t o_cand = take(8ull * pool * CAND_CAP);
  const size_t o_flags = take(4ull * max_batch);
  const size_t o_stats = take(16ull * max_batch);
  const size_t o_skeys = take(8ull * SLOW_WGS * 3 * max_vocab);
  const size_t o_sp = take(4ull * SLOW_WGS * max_vocab);
  const size_t o_si = take(4ull * SLOW_WGS * max_vocab);
  const size_t o_status = take(256);
  void* mem = nullptr;
  HIPCHK(hipMalloc(&mem, off));
  hipError_t e = hipMemset(mem, 0, off);
  if (e != hipSuccess) {
    (void)hipFree(mem);
    return fail(LLMK_ERR_HIP, std::string("hipMemset failed: ") + hipGetErrorString(e));
  }
  e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    (void)hipFree(mem);
    return fail(LLMK_ERR_HIP, std::string("hipDeviceSynchronize failed: ") + hipGetErrorString(e));
  }
  char* base = (char*)mem;
  llmk_sampler* s = new llmk_sampler();
  s->device = device;
  s->max_batch = max_batch;
  s->max_vocab = max_vocab;
  s->mem = mem;
  s->mem_bytes = off;
  s->ws.row_arrive = (uint32_t*)(base + o_arrive);
  s->ws.tile_part = (float2*)(base + o_part);
  s->ws.seg_meta = (uint4*)(base + o_meta);
  s->ws.cand = (uint2*)(base + o_cand);
  s->ws.row_flags = (uint32_t*)(base + o_flags);
  s->ws.row_stats = (float4*)(base + o_stats);
  s->ws.slow_keys = (uint64_t*)(base + o_skeys);
  s->ws.slow_p = (float*)(base + o_sp);
  s->ws.slow_idx = (uint32_t*)(base + o_si);
  s->ws.status = (uint32_t*)(base + o_status);
  s->ws.max_vocab = max_vocab;
  *out = s;
  g_last_error.clear();
  return LLMK_OK;
}

extern "C" void llmk_sampler_destroy(llmk_sampler* s) {
  if (!s) return;
  (void)hipSetDevice(s->device);
  (void)hipDeviceSynchronize();
  (void)hipFree(s->mem);
  delete s;
}

extern "C" int llmk_sampler_status(llmk_sampler* s, void* stream,
                                   uint32_t* status) {
  if (!s || !status) return fail(LLMK_ERR_INVALID_ARGUMENT, "NULL argument");
  HIPCHK(hipSetDevice(s->device));
  hipStream_t st = (hipStream_t)stream;
  uint32_t v = 0;
  HIPCHK(hipMemcpyAsync(&v, s->ws.status, 4, hipMemcpyDeviceToHost, st));
  HIPCHK(hipMemsetAsync(s->ws.status, 0, 4, st));
  HIPCHK(hipStreamSynchronize(st));
  *status = v;
  return LLMK_OK;
}

extern "C" int llmk_sample_batch(llmk_sampler* s,
                                 const llmk_sample_batch_args* in,
                                 void* stream) {
  if (!s) return fail(LLMK_ERR_INVALID_ARGUMENT, "sampler is NULL");
  if (!in) return fail(LLMK_ERR_INVALID_ARGUMENT, "args is NULL");
  if (in->vocab == 0) return fail(LLMK_ERR_EMPTY_LOGITS, "Empty logits passed to sampler");
  if (in->batch == 0) return fail(LLMK_ERR_INVALID_ARGUMENT, "batch is 0");
  if (!in->logits || !in->out_tokens || !in->uniforms)
    return fail(LLMK_ERR_INVALID_ARGUMENT, "logits, uniforms and out_tokens are required");
  if (in->dtype != LLMK_F32 && in->dtype != LLMK_BF16)
    return fail(LLMK_ERR_INVALID_ARGUMENT, "dtype must be LLMK_F32 or LLMK_BF16");
  if (in->batch > s->max_batch || in->vocab > s->max_vocab)
    return fail(LLMK_ERR_CAPACITY, "batch or vocab above the sampler's maxima");
  if (in->row_stride < in->vocab)
    return fail(LLMK_ERR_INVALID_ARGUMENT, "row_stride < vocab");
  if ((in->hist_offsets == nullptr) != (in->hist_tokens == nullptr))
    return fail(LLMK_ERR_INVALID_ARGUMENT, "hist_offsets and hist_tokens go together");
  if (in->allow_mask && in->mask_words_per_row < (in->vocab + 31) / 32)
    return fail(LLMK_ERR_INVALID_ARGUMENT, "mask_words_per_row < ceil(vocab/32)");
  if (in->out_cap && !in->out_ids && !in->out_probs)
    return fail(LLMK_ERR_INVALID_ARGUMENT, "out_cap without out_ids/out_probs");
  const size_t esz = in->dtype == LLMK_F32 ? 4 : 2;
  const size_t align = in->dtype == LLMK_F32 ? 16 : 8;
  if (((uintptr_t)in->logits % align) != 0 || ((in->row_stride * esz) % align) != 0)
    return fail(LLMK_ERR_ALIGNMENT, "logit rows must be 16-byte (fp32) / 8-byte (bf16) aligned");

  Args a;
  a.logits = in->logits;
  a.dtype = in->dtype;
  a.B = in->batch;
  a.V = in->vocab;
  a.stride = in->row_stride;
  a.T = in->temperature;
  a.top_p = in->top_p;
  a.min_p = in->min_p;
  a.rp = in->repetition_penalty;
  a.pp = in->presence_penalty;
  a.fp = in->frequency_penalty;
  a.top_k = in->top_k;
  a.hoff = in->hist_offsets;
  a.htok = in->hist_tokens;
  a.mask = in->allow_mask;
  a.mask_words = in->mask_words_per_row;
  a.u = in->uniforms;
  a.out_tok = in->out_tokens;
  a.out_ids = in->out_ids;
  a.out_cnt = in->out_count;
  a.out_probs = in->out_probs;
  a.out_cap = in->out_cap;
  a.ntiles = (a.V + TILE - 1) / TILE;
  // Segments per row: enough workgroups to cover the 256 CUs, at least 4
  // tiles per segment.
  uint32_t G = (256 + a.B - 1) / a.B;
  const uint32_t gmax = (a.ntiles + 3) / 4;
  if (G > gmax) G = gmax;
  if (G < 1) G = 1;
  while ((uint64_t)a.B * G > (s->max_batch > MAX_WGS ? s->max_batch : MAX_WGS)) --G;
  a.tps = (a.ntiles + G - 1) / G;
  a.G = (a.ntiles + a.tps - 1) / a.tps;
  a.xcd_map = (a.G > 1 && (a.B % 8) == 0) ? 1u : 0u;

  HIPCHK(hipSetDevice(s->device));
  hipStream_t st = (hipStream_t)stream;
  const size_t lds_stream =
      4 * (stream_lds_words(a.tps) > finalize_lds_words() ? stream_lds_words(a.tps)
                                                          : finalize_lds_words());
  const dim3 grid(a.B * a.G), block(NT);
  if (a.dtype == LLMK_F32)
    hipLaunchKernelGGL(stream_kernel<LLMK_F32>, grid, block, lds_stream, st, a, s->ws);
  else
    hipLaunchKernelGGL(stream_kernel<LLMK_BF16>, grid, block, lds_stream, st, a, s->ws);
  HIPCHK(hipGetLastError());
  const uint32_t nslow = a.B < SLOW_WGS ? a.B : SLOW_WGS;
  const size_t lds_slow = slow_lds_bytes(a.V);
  if (a.dtype == LLMK_F32)
    hipLaunchKernelGGL(slow_kernel<LLMK_F32>, dim3(nslow), dim3(SLOW_NT), lds_slow, st, a, s->ws);
  else
    hipLaunchKernelGGL(slow_kernel<LLMK_BF16>, dim3(nslow), dim3(SLOW_NT), lds_slow, st, a, s->ws);
  HIPCHK(hipGetLastError());
  return LLMK_OK;
}
