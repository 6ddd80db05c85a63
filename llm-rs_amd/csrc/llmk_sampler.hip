// llmk_sampler.hip — MI355X (gfx950) batched token sampling for llm-rs.
//
// Replaces the host loop llm-scheduler/src/scheduler.rs:138-145, which calls
// llm-core/src/sampler.rs:25-125 (sample_logits) once per row, with one
// stream-ordered call that samples the whole batch on the GPU.
//
// One kernel, `stream_kernel`, one workgroup per (row, vocabulary segment):
//   * history  the row's token history restricted to the segment becomes an
//              LDS bitmap + popcount prefix (rank of a token among the
//              history's distinct tokens) and a table of the penalised logits
//              of those tokens (repetition, presence, frequency).
//   * stream   the segment's logits are read once from HBM with 128-bit
//              non-temporal loads in 1024-token tiles: an fp32 lane owns 4
//              runs of 4 consecutive tokens, a bf16/f16 lane 2 runs of 8
//              (one 16-byte load per run).  Per tile: history
//              tokens take their penalised value, the allow-mask applies, and
//              the wave computes the tile max (or the tile argmax for greedy
//              rows) and appends top candidates above a rising threshold
//              kept in an LDS histogram of the logits' order-preserving keys.
//   * finalize the last workgroup of the row (arrival counter when a row spans
//              several workgroups) merges the tile maxima, takes the
//              normaliser S, computes exact probabilities of the candidates,
//              ranks them by (p desc, idx asc), proves no other token can
//              precede the ones used, and runs min-p / top-k / top-p / the
//              draw exactly as sampler.rs:77-124.  Rows without top-k use the
//              reference's sequential f32 S (the exact normaliser); top-k
//              rows take S = 1 only where a rounding-band check proves every
//              decision (min-p cut, top-k set, top-p cut, draw) to be the
//              reference's whatever S is, else the exact S and a rerun: the
//              launch after this one (phase 1, xs_phase) sums that S over
//              the row's 16384-element windows on many workgroups, and the
//              last of them runs the row's candidate path again.
//   * slow     rows the candidate path cannot prove exact (top-k = 0 with a
//              large nucleus, candidate overflow, fully masked rows) are done
//              by the same workgroup: exact probabilities of the whole row,
//              a stable LSD radix sort in a global scratch slot, and the same
//              sequential semantics.  Rows whose history outgrows the LDS
//              rank tables take it over logits penalised and materialised in
//              the slot.
//
// Rows that do not start 16-byte aligned are first copied to aligned rows of
// a staging buffer (realign_kernel).
//
// Numerics are fixed (llmk_numerics.h); the CPU mirror oracle restates them.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "llmk_numerics.h"
#include "llmk_sampler.h"

namespace llmk {

// Explicit address spaces: LDS (3) and global (1).  Pointers that pass
// through structs or function parameters would otherwise become generic
// (flat) pointers, whose loads wait on both the vector-memory and the LDS
// counters.
#define LDS __attribute__((address_space(3)))
#define GLB __attribute__((address_space(1)))
template <class T>
__device__ __forceinline__ GLB T* G(T* p) { return (GLB T*)p; }
template <class T>
__device__ __forceinline__ const GLB T* G(const T* p) { return (const GLB T*)p; }

typedef float f2v __attribute__((ext_vector_type(2)));
typedef float f4v __attribute__((ext_vector_type(4)));
typedef uint32_t u2v __attribute__((ext_vector_type(2)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));

constexpr uint32_t TILE = 1024;      // canonical vocabulary tile
constexpr int WAVE = 64;
constexpr int NW = 16;               // waves per workgroup
constexpr int NT = NW * WAVE;        // 1024 threads
constexpr uint32_t NBINS = 4096;     // fine histogram bins: key >> 20
constexpr uint32_t BIN_SHIFT = 20;
constexpr uint32_t CBIN_SHIFT = 26;  // coarse bins: key >> 26 (64 bins)
constexpr uint32_t U_MAX = 8192;     // distinct history tokens per segment
constexpr uint32_t CAND_CAP = 8192;  // candidate entries per workgroup
constexpr uint32_t SORT_CAP = 4096;  // candidates sorted in finalize
constexpr uint32_t KMAX = 1024;      // largest top-k served by the fast path
constexpr uint32_t KCAND_NOK = 1024; // candidate target when top-k is off
constexpr uint32_t MAX_TILES = 1024; // max_vocab <= 2^20
constexpr uint32_t CHUNK_TILES = 16;  // tiles per history chunk (segments are whole chunks)
constexpr uint32_t MAX_CHUNKS = MAX_TILES / CHUNK_TILES;
constexpr uint32_t MAX_SLOTS = MAX_TILES + MAX_CHUNKS;  // partials per row: tiles, then chunks
constexpr uint32_t LCAP = 1024;       // candidates a single-segment row keeps in LDS
constexpr uint32_t MAX_SEG = 64;     // segments per row
constexpr uint32_t MAX_WGS = 4096;   // candidate-buffer pool entries
constexpr uint32_t SLOW_SLOTS = 512;  // most global scratch slots of the slow path
constexpr uint32_t SLOW_BINS = 2048; // slow path: bins of the processed logits
constexpr uint32_t EMPTY = 0xffffffffu;
constexpr float NEG_INF = -__builtin_huge_valf();
constexpr float LOG2E_F = 0x1.715476p+0f;  // the slow path's bins of (l - L)/T, in octaves
// The exact S of rows that fail the band check, on many workgroups (phase 1)
constexpr uint32_t XS_JOBS = 8;                        // rows per call
constexpr uint32_t XS_W = 16 * TILE;                   // a window: 16 segments of a tile
constexpr uint32_t XS_SAVE = 2 * MAX_SLOTS + 2 * LCAP;  // LDS partials + candidates
constexpr uint32_t XS_JOB_WORDS = 32;
constexpr uint32_t XS_PRE = 2 + XS_JOBS;                // xs_ctl: window 0's (sum, tag) per job
constexpr uint32_t XS_CTL_WORDS = XS_PRE + 2 * XS_JOBS;

// Words a workgroup passes from one phase to the next past the dynamic
// shared memory, which each phase lays out afresh (static LDS).
__shared__ uint32_t g_bcast[4];

enum : uint32_t { MODE_INVALID = 0, MODE_GREEDY = 1, MODE_SAMPLE = 2 };
enum : uint32_t { FLAG_OVERFLOW = 1u, FLAG_HIST_OVERFLOW = 2u, FLAG_NAN = 4u };

struct Args {
  const void* logits;
  int32_t dtype;
  float sc_m1, sc_cap;  // softcap: 1/cap and cap in the logits' dtype (DT & SOFTCAP)
  uint32_t B, V;
  uint64_t stride;
  const float *T, *top_p, *min_p, *rp, *pp, *fp;
  const int32_t* top_k;
  const uint32_t *hoff, *htok, *mask;
  const uint32_t* hlen;  // optional: row b's history is htok[hoff[b] .. hoff[b] + hlen[b])
  const uint32_t* hcnt;  // optional: occurrences of each htok entry (the count-table form)
  uint32_t mask_words;
  const float* u;
  uint32_t *out_tok, *out_ids, *out_cnt;
  float* out_probs;
  uint32_t out_cap;
  uint32_t G, tps, ntiles, nchunks;
  // single-segment rows: LDS word offsets of the kept partials (MAX_SLOTS
  // f2v) and candidates (LCAP u2v), past both the stream and finalize layouts
  uint32_t lds_part, lds_cand;
  uint32_t xcd_map;  // 1: the segments of a row share an XCD
  // apply_top_p: per row, the last kept entry's index, the kept count and
  // the m and S its probabilities used; top_p clamped to [0, 1], NaN read as 1
  // (the mask form's no-op, not an invalid row)
  u4v* cut;
  uint32_t tp_clamp;
  // 0: the sampling launch; 1: the launch after it that sums the reference's
  // S, window by window on many workgroups, for the rows whose band check
  // failed (up to xs_cap rows per call; the sampling launch does the rest
  // itself)
  uint32_t phase, xs_cap;
  uint32_t xs_lds;  // phase 1's dynamic LDS in words
  // the call's parity: its jobs are counted in xs_ctl[epoch & 1], and its
  // sampling launch clears the other count for the next call
  uint32_t epoch;
  // phase 1's bounded waits (for the sums of earlier windows, for window
  // 0's own walk): at most this many polls (XS_SPIN; a test sets 0 to take
  // the paths where a wait runs out)
  uint32_t xs_spin;
};

struct Ws {
  uint32_t* row_arrive;  // [max_batch]
  f2v* tile_part;        // [max_batch][MAX_SLOTS]: max, sum (or first argmax) per slot
  u4v* seg_meta;         // [pool]: count, beta, flags, -
  u2v* cand;             // [pool][CAND_CAP]: value bits, index
  uint32_t* slow_lock;   // [slow_slots]
  uint64_t* slow_keys;   // [slow_slots][3][max_vocab]
  float* slow_p;         // [slow_slots][max_vocab]
  uint32_t* slow_idx;    // [slow_slots][max_vocab]
  uint32_t* status;      // [1]
  u4v* cut;              // [max_batch]: apply_top_p's cut per row
  uint32_t* mtok;        // [max_batch]: apply_top_p's (unused) draws
  float* zu;             // [max_batch]: zeros, its uniforms
  // the exact S of deferred rows (phase 1): jobs posted, workgroups done and
  // per job its arrival count; the jobs; per job and window its sum and that
  // sum's flag; per job and segment its pairs and terms; per job the
  // single-segment row's LDS partials and candidates
  uint32_t* xs_ctl;      // [XS_CTL_WORDS]: job counts of even / odd calls, arrivals,
                         // window 0's (sum, tag) per job
  uint32_t* xs_job;      // [XS_JOBS][XS_JOB_WORDS]
  float* xs_wsum;        // [XS_JOBS][xs_maxw]
  uint32_t* xs_wflag;    // [XS_JOBS][xs_maxw]
  uint32_t* xs_meta;     // [XS_JOBS][xs_maxw * 16][8]
  float* xs_terms;       // [XS_JOBS][xs_maxw * 16][TILE]
  uint32_t* xs_runs;     // [XS_JOBS][xs_maxw * 16][XS_RUNW]
  uint32_t* xs_save;     // [XS_JOBS][XS_SAVE]
  uint32_t xs_maxw;
  uint32_t max_vocab;
  uint32_t slow_slots;   // min(max_batch, SLOW_SLOTS): rows b, b + slow_slots, ... share one
};

struct RowP {
  float T, top_p, min_p, rp, pp, fp;
  int32_t K;
  uint32_t mode;
  uint32_t Kc;  // candidate target; 0 = candidate path impossible
};

__device__ __forceinline__ bool finitef(float x) { return __builtin_isfinite(x); }

// Defaults of absent per-row arrays (SampleParams, llm-core/src/types.rs:
// 186-195), read in place of the array: every load is then unconditional.
__constant__ float kOneF = 1.0f;
__constant__ uint32_t kZeroU = 0u;
template <class T>
__device__ __forceinline__ const T* row_or(const T* p, uint32_t b, const void* dflt) {
  return p ? p + b : (const T*)dflt;
}

// The row's parameters, uniform, history extent and uniform as loaded: all
// requested together, before anything branches on one of them, so that they
// cost one round trip.
struct RowIn {
  float T, top_p, min_p, rp, pp, fp, u;
  int32_t K;
  uint32_t h0, hn, hl;
};
__device__ __forceinline__ RowIn load_row(const Args& a, uint32_t b) {
  RowIn r;
  r.T = *G(row_or(a.T, b, &kOneF));
  r.top_p = *G(row_or(a.top_p, b, &kOneF));
  r.min_p = *G((const float*)row_or(a.min_p, b, &kZeroU));
  r.rp = *G(row_or(a.rp, b, &kOneF));
  r.pp = *G((const float*)row_or(a.pp, b, &kZeroU));
  r.fp = *G((const float*)row_or(a.fp, b, &kZeroU));
  r.K = *G((const int32_t*)row_or(a.top_k, b, &kZeroU));
  r.u = *G(a.u + b);
  r.h0 = *G(row_or(a.hoff, b, &kZeroU));
  r.hn = *G(row_or(a.hoff, b + 1, &kZeroU));
  r.hl = *G(row_or(a.hlen, b, &kZeroU));
  return r;
}

__device__ __forceinline__ RowP row_params(const Args& a, const RowIn& in) {
  RowP r;
  r.T = in.T;
  r.top_p = in.top_p;
  if (a.tp_clamp) r.top_p = r.top_p < 0.0f ? 0.0f : (r.top_p < 1.0f ? r.top_p : 1.0f);
  r.min_p = in.min_p;
  r.rp = in.rp;
  r.pp = in.pp;
  r.fp = in.fp;
  r.K = in.K;
  const bool bad = !finitef(r.T) || r.K < 0 || !finitef(r.top_p) ||
                   !finitef(r.min_p) || !(r.min_p >= 0.0f) || !finitef(r.rp) ||
                   !finitef(r.pp) || !finitef(r.fp);
  r.mode = bad ? MODE_INVALID : (r.T <= 1e-5f ? MODE_GREEDY : MODE_SAMPLE);
  const bool topk_on = r.K > 0 && (uint32_t)r.K < a.V;
  // top-k rows gather one candidate past the K-th (the band check compares
  // the two)
  r.Kc = topk_on ? ((uint32_t)r.K <= KMAX ? (uint32_t)r.K + 1u : 0u) : KCAND_NOK;
  return r;
}

// ---------------------------------------------------------------------------
// Wave64 helpers on DPP (row_shr within 16-lane rows, row_bcast across rows)
// ---------------------------------------------------------------------------
template <int CTRL, int RM, bool BC>
__device__ __forceinline__ float dppf(float old, float src) {
  return __int_as_float(__builtin_amdgcn_update_dpp(
      __float_as_int(old), __float_as_int(src), CTRL, RM, 0xf, BC));
}
template <int CTRL, int RM, bool BC>
__device__ __forceinline__ uint32_t dppu(uint32_t old, uint32_t src) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)src, CTRL, RM, 0xf, BC);
}
__device__ __forceinline__ uint32_t umax_(uint32_t a, uint32_t b) { return a > b ? a : b; }
__device__ __forceinline__ float bcast63f(float x) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 63));
}
__device__ __forceinline__ uint32_t bcast63u(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
}

// Sum of lanes 0..63 as a balanced binary tree over contiguous lanes
// ((x0+x1)+(x2+x3))+...; the root forms in lane 63 and is broadcast.
__device__ __forceinline__ float wave_tree_sum(float x) {
  x = x + dppf<0x111, 0xf, true>(0.0f, x);
  x = x + dppf<0x112, 0xf, true>(0.0f, x);
  x = x + dppf<0x114, 0xf, true>(0.0f, x);
  x = x + dppf<0x118, 0xf, true>(0.0f, x);
  x = x + dppf<0x142, 0xa, false>(0.0f, x);
  x = x + dppf<0x143, 0xc, false>(0.0f, x);
  return bcast63f(x);
}
// Maximum over the lanes of x (never NaN): on order-preserving keys, whose
// maximum needs no NaN handling, so each step is one v_max_u32 with DPP;
// lanes outside a row read 0, the smallest key.
__device__ __forceinline__ float wave_max(float x) {
  const uint32_t b = __float_as_uint(x);
  uint32_t k = b ^ ((uint32_t)((int32_t)b >> 31) | 0x80000000u);
  k = umax_(k, dppu<0x111, 0xf, true>(0u, k));
  k = umax_(k, dppu<0x112, 0xf, true>(0u, k));
  k = umax_(k, dppu<0x114, 0xf, true>(0u, k));
  k = umax_(k, dppu<0x118, 0xf, true>(0u, k));
  k = umax_(k, dppu<0x142, 0xa, true>(0u, k));
  k = umax_(k, dppu<0x143, 0xc, true>(0u, k));
  const uint32_t r = bcast63u(k);
  return __uint_as_float((r & 0x80000000u) ? (r & 0x7fffffffu) : ~r);
}
__device__ __forceinline__ uint32_t umin(uint32_t a, uint32_t b) { return a < b ? a : b; }
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t x) {
  x = umin(x, dppu<0x111, 0xf, false>(x, x));
  x = umin(x, dppu<0x112, 0xf, false>(x, x));
  x = umin(x, dppu<0x114, 0xf, false>(x, x));
  x = umin(x, dppu<0x118, 0xf, false>(x, x));
  x = umin(x, dppu<0x142, 0xa, false>(x, x));
  x = umin(x, dppu<0x143, 0xc, false>(x, x));
  return bcast63u(x);
}
__device__ __forceinline__ uint32_t umax(uint32_t a, uint32_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
  x = umax(x, dppu<0x111, 0xf, true>(0u, x));
  x = umax(x, dppu<0x112, 0xf, true>(0u, x));
  x = umax(x, dppu<0x114, 0xf, true>(0u, x));
  x = umax(x, dppu<0x118, 0xf, true>(0u, x));
  x = umax(x, dppu<0x142, 0xa, true>(0u, x));
  x = umax(x, dppu<0x143, 0xc, true>(0u, x));
  return bcast63u(x);
}
// Inclusive prefix sum over lanes.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x) {
  x += dppu<0x111, 0xf, true>(0u, x);
  x += dppu<0x112, 0xf, true>(0u, x);
  x += dppu<0x114, 0xf, true>(0u, x);
  x += dppu<0x118, 0xf, true>(0u, x);
  x += dppu<0x142, 0xa, false>(0u, x);
  x += dppu<0x143, 0xc, false>(0u, x);
  return x;
}
__device__ __forceinline__ uint32_t lanes_below(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Block-wide exclusive scan of one value per thread (NT threads).
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t x, LDS uint32_t* red, uint32_t& total) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const uint32_t incl = wave_incl_scan(x);
  if (lane == 63) red[wv] = incl;
  __syncthreads();
  uint32_t off = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const uint32_t c = red[i];
    off += (i < wv) ? c : 0u;
    tot += c;
  }
  __syncthreads();
  total = tot;
  return off + incl - x;
}
__device__ __forceinline__ float block_max(float x, LDS float* red) {
  x = wave_max(x);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  if (lane == 0) red[wv] = x;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) r = fmaxf(r, red[i]);
  __syncthreads();
  return r;
}
__device__ __forceinline__ uint32_t block_min_u32(uint32_t x, LDS uint32_t* red) {
  x = wave_min_u32(x);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  if (lane == 0) red[wv] = x;
  __syncthreads();
  uint32_t r = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) r = umin(r, red[i]);
  __syncthreads();
  return r;
}

// Wait until this wave's global stores have reached L2 (vmcnt(0)).
__device__ __forceinline__ void wait_stores() { __builtin_amdgcn_s_waitcnt(0x0f70); }

// ---------------------------------------------------------------------------
// History: bitmap over a vocabulary range, popcount prefix, penalised values
// ---------------------------------------------------------------------------
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

// A 16-bit logit (bf16 or f16 bits) as f32, exactly.
template <int DT>
__device__ __forceinline__ float cvt16(uint32_t h) {
  if ((DT & 3) == LLMK_BF16) return __uint_as_float(h << 16);
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// Template flag on the dtype: the logits are the lm_head output before
// final_logit_softcapping, capped as they are read.  1/cap and cap (in the
// logits' dtype) sit in LDS, written before the kernel's first barrier.
constexpr int SOFTCAP = 4;
__shared__ float g_softcap[2];
// f32 -> the logits' dtype, round to nearest even (NaN stays NaN)
template <int DT>
__device__ __forceinline__ float round_dt(float x) {
  if ((DT & 3) == LLMK_BF16) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return __uint_as_float((u | 0x00400000u) & 0xffff0000u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return __uint_as_float(u & 0xffff0000u);
  }
  if ((DT & 3) == LLMK_F16) return (float)(_Float16)x;
  return x;
}
// final_logit_softcapping as candle evaluates it on the logits tensor
// (candle.rs:1803-1807): (x / cap).tanh() * cap, where dividing or
// multiplying a tensor by a scalar is its affine map x * m + 0 (m = 1/cap or
// cap, as the dtype) and tanh is glibc's tanhf; in a 16-bit dtype every
// operation rounds to it.
template <int DT>
__device__ __forceinline__ float softcap(float x) {
  if (!(DT & SOFTCAP)) return x;
  float y = round_dt<DT>(x * g_softcap[0]);
  y = round_dt<DT>(y + 0.0f);
  float t = round_dt<DT>(tanh_ref(y));
  t = round_dt<DT>(t * g_softcap[1]);
  return round_dt<DT>(t + 0.0f);
}
template <int DT>
__device__ __forceinline__ void softcap_init(const Args& a) {
  if (DT & SOFTCAP)
    if (threadIdx.x < 2) g_softcap[threadIdx.x] = threadIdx.x ? a.sc_cap : a.sc_m1;
}

template <int DT>
__device__ __forceinline__ float load_logit(const void* row, uint32_t e) {
  if ((DT & 3) == LLMK_F32) return softcap<DT>(G((const float*)row)[e]);
  return softcap<DT>(cvt16<DT>(G((const uint16_t*)row)[e]));
}

struct Hist {
  LDS uint32_t* bitmap;  // nwords
  LDS uint16_t* pre;     // nwords: distinct history tokens in words before
  LDS float* pen;        // U_MAX: penalised logit by rank (counts while building)
  LDS uint32_t* tokr;    // U_MAX: token of each rank
  uint32_t lo;
  __device__ __forceinline__ uint32_t rank(uint32_t t) const {
    const uint32_t o = t - lo, w = o >> 5;
    return pre[w] + __popc(bitmap[w] & ((1u << (o & 31)) - 1u));
  }
};

__host__ __device__ inline size_t hist_lds_words(uint32_t nwords) {
  return (size_t)((nwords + 3) & ~3u) + (size_t)(((nwords + 1) / 2 + 3) & ~3u) + 2 * U_MAX;
}
__device__ __forceinline__ void hist_carve(Hist& h, LDS uint32_t* base, uint32_t nwords) {
  h.bitmap = base;
  h.pre = (LDS uint16_t*)(base + ((nwords + 3) & ~3u));
  h.pen = (LDS float*)(base + ((nwords + 3) & ~3u) + (((nwords + 1) / 2 + 3) & ~3u));
  h.tokr = (LDS uint32_t*)(h.pen + U_MAX);
}

// Ranks of the segment's history tokens once its bitmap is complete, built
// by the first nw waves, which call sync() together twice (the second time
// at the end).  Thread i of them owns a contiguous run of bitmap words: the
// run's popcount, an exclusive scan over the threads, then pre[w] = history
// tokens in the words before w and tokr[r] = the token of rank r (tokens in
// increasing order).  Tokens of rank >= U_MAX are cleared from the bitmap
// and the overflow flag is raised: they are then ordinary, unpenalised
// tokens.  Returns the number of ranks (<= U_MAX).  wtot: nw words.
template <class Sync>
__device__ __forceinline__ uint32_t build_ranks(const Hist& h, uint32_t nwords,
                                                LDS uint32_t* wtot, LDS uint32_t* flags,
                                                uint32_t nw, Sync& sync) {
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wv = tid >> 6;
  const uint32_t per = (nwords + 64u * nw - 1u) / (64u * nw);
  const uint32_t w0 = tid * per < nwords ? tid * per : nwords;
  const uint32_t w1 = w0 + per < nwords ? w0 + per : nwords;
  // runs of up to 8 words are read at once (taken branches cost a lone
  // wave more than the reads)
  uint32_t c = 0;
  for (uint32_t b0 = w0; b0 < w1; b0 += 8) {
    uint32_t x[8];
#pragma unroll
    for (uint32_t q = 0; q < 8; ++q) x[q] = b0 + q < w1 ? h.bitmap[b0 + q] : 0u;
#pragma unroll
    for (uint32_t q = 0; q < 8; ++q) c += (uint32_t)__popc(x[q]);
  }
  const uint32_t incl = wave_incl_scan(c);
  if (lane == 63) wtot[wv] = incl;
  sync();
  uint32_t r = incl - c, total = 0;
  for (uint32_t i = 0; i < nw; ++i) {
    const uint32_t t = wtot[i];
    r += i < wv ? t : 0u;
    total += t;
  }
  for (uint32_t b0 = w0; b0 < w1; b0 += 8) {
    uint32_t x[8];
#pragma unroll
    for (uint32_t q = 0; q < 8; ++q) x[q] = b0 + q < w1 ? h.bitmap[b0 + q] : 0u;
#pragma unroll
    for (uint32_t q = 0; q < 8; ++q) {
      const uint32_t wi = b0 + q;
      uint32_t bits = x[q];
      const uint32_t cw = (uint32_t)__popc(bits);
      if (wi < w1) h.pre[wi] = (uint16_t)(r < U_MAX ? r : U_MAX);
      if (wi < w1 && r + cw > U_MAX) {  // keep the first U_MAX - r tokens of the word
        const uint32_t keep = r < U_MAX ? U_MAX - r : 0u;
        uint32_t kept = 0, rest = bits;
        for (uint32_t k = 0; k < keep; ++k) {
          kept |= rest & (0u - rest);
          rest &= rest - 1u;
        }
        bits = kept;
        h.bitmap[wi] = kept;
      }
      // two tokens per step
      while (bits) {
        const uint32_t b1 = (uint32_t)__builtin_ctz(bits);
        bits &= bits - 1u;
        h.tokr[r++] = h.lo + 32u * wi + b1;
        if (bits) {
          const uint32_t b2 = (uint32_t)__builtin_ctz(bits);
          bits &= bits - 1u;
          h.tokr[r++] = h.lo + 32u * wi + b2;
        }
      }
    }
  }
  if (total > U_MAX && tid == 0) __atomic_fetch_or(flags, FLAG_HIST_OVERFLOW, __ATOMIC_RELAXED);
  sync();
  return total < U_MAX ? total : U_MAX;
}

// pre[w] = history tokens in the bitmap words before w, built by the first nw
// waves from contiguous runs of words (a popcount per run, an exclusive scan
// over the threads), which call sync() together twice.  Returns the number
// of tokens, which the caller knows to be at most U_MAX.  wtot: nw words.
template <class Sync>
__device__ __forceinline__ uint32_t build_pre(const Hist& h, uint32_t nwords,
                                              LDS uint32_t* wtot, uint32_t nw, Sync& sync) {
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wv = tid >> 6;
  const uint32_t per = (nwords + 64u * nw - 1u) / (64u * nw);
  const uint32_t w0 = tid * per < nwords ? tid * per : nwords;
  const uint32_t w1 = w0 + per < nwords ? w0 + per : nwords;
  uint32_t c = 0;
  for (uint32_t b0 = w0; b0 < w1; b0 += 8) {
    uint32_t x[8];
#pragma unroll
    for (uint32_t q = 0; q < 8; ++q) x[q] = b0 + q < w1 ? h.bitmap[b0 + q] : 0u;
#pragma unroll
    for (uint32_t q = 0; q < 8; ++q) c += (uint32_t)__popc(x[q]);
  }
  const uint32_t incl = wave_incl_scan(c);
  if (lane == 63) wtot[wv] = incl;
  sync();
  uint32_t r = incl - c, total = 0;
  for (uint32_t i = 0; i < nw; ++i) {
    const uint32_t t = wtot[i];
    r += i < wv ? t : 0u;
    total += t;
  }
  for (uint32_t b0 = w0; b0 < w1; b0 += 8) {
    uint32_t x[8];
#pragma unroll
    for (uint32_t q = 0; q < 8; ++q) x[q] = b0 + q < w1 ? h.bitmap[b0 + q] : 0u;
#pragma unroll
    for (uint32_t q = 0; q < 8; ++q) {
      if (b0 + q < w1) h.pre[b0 + q] = (uint16_t)r;
      r += (uint32_t)__popc(x[q]);
    }
  }
  sync();
  return total;
}

// A barrier among waves 0 .. n-1 while the others run on: an arrival count
// in LDS that the waiting waves poll.  Every one of the n waves makes every
// call, and none of them waits on the other waves in between, so each wait
// ends.
struct GroupSync {
  LDS uint32_t* ctr;
  uint32_t n, gen;
  __device__ __forceinline__ void operator()() {
    ++gen;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if ((threadIdx.x & 63u) == 0) __atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED);
    while (__atomic_load_n(ctr, __ATOMIC_RELAXED) < n * gen) __builtin_amdgcn_s_sleep(1);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  }
};
struct BarrierSync {
  __device__ __forceinline__ void operator()() { __syncthreads(); }
};

// Builds the history tables for tokens in [lo, hi) of row b.  All threads.
// Global round trips: the row's history (held in registers, HTPT tokens per
// thread per pass) and one gather of the logits of the distinct tokens.
// Occurrences of history entry i: its count in the count-table form (read
// as at least 1: a listed token is in the history), else 1 per entry.
__device__ __forceinline__ uint32_t hist_weight(const Args& a, uint32_t i) {
  return a.hcnt ? umax(G(a.hcnt)[i], 1u) : 1u;
}

constexpr int HTPT = 8;
template <int DT>
__device__ __forceinline__ void build_history(const Args& a, const RowP& P, uint32_t b,
                              const void* row, uint32_t lo, uint32_t hi,
                              uint32_t nwords, Hist& h, LDS uint32_t* red,
                              LDS uint32_t* flags) {
  const uint32_t tid = threadIdx.x;
  const bool need_pen = P.rp != 1.0f || P.pp != 0.0f || P.fp != 0.0f;
  const bool have = need_pen && a.hoff;
  const uint32_t h0 = have ? G(a.hoff)[b] : 0u;
  const uint32_t h1 = have ? (a.hlen ? h0 + G(a.hlen)[b] : G(a.hoff)[b + 1]) : 0u;
  uint32_t tk[HTPT];
#pragma unroll
  for (int q = 0; q < HTPT; ++q) {
    const uint32_t i = h0 + q * NT + tid;
    tk[q] = (i < h1) ? G(a.htok)[i] : EMPTY;
  }
  for (uint32_t i = tid; i < nwords; i += NT) h.bitmap[i] = 0;
  __syncthreads();
  if (!have) {  // uniform; the tables stay empty
    for (uint32_t i = tid; i < nwords; i += NT) h.pre[i] = 0;
    __syncthreads();
    return;
  }
  const bool need_cnt = P.fp != 0.0f;
  const bool one_pass = h1 - h0 <= (uint32_t)(HTPT * NT);
  for (uint32_t c0 = h0; c0 < h1; c0 += HTPT * NT) {
#pragma unroll
    for (int q = 0; q < HTPT; ++q) {
      uint32_t t = tk[q];
      if (c0 != h0) {
        const uint32_t i = c0 + q * NT + tid;
        t = (i < h1) ? G(a.htok)[i] : EMPTY;
      }
      if (t >= lo && t < hi) __atomic_fetch_or(&h.bitmap[(t - lo) >> 5], 1u << (t & 31), __ATOMIC_RELAXED);
    }
  }
  __syncthreads();
  // exclusive popcount prefix over the words, each thread a contiguous run;
  // the token of every rank is recorded
  const uint32_t wpt = (nwords + NT - 1) / NT;
  const uint32_t w0 = tid * wpt, w1 = (w0 + wpt < nwords) ? w0 + wpt : nwords;
  uint32_t local = 0;
  for (uint32_t wi = w0; wi < w1; ++wi) local += __popc(h.bitmap[wi]);
  uint32_t U;
  uint32_t run = block_excl_scan(local, red, U);
  for (uint32_t wi = w0; wi < w1; ++wi) {
    h.pre[wi] = (uint16_t)(run < 0xffffu ? run : 0xffffu);
    uint32_t bits = h.bitmap[wi];
    while (bits) {
      const uint32_t bit = __builtin_ctz(bits);
      bits &= bits - 1;
      if (run < U_MAX) h.tokr[run] = lo + 32 * wi + bit;
      ++run;
    }
  }
  if (U > U_MAX && tid == 0) __atomic_fetch_or(flags, FLAG_HIST_OVERFLOW, __ATOMIC_RELAXED);
  const uint32_t Uc = U < U_MAX ? U : U_MAX;
  LDS uint32_t* cnt = (LDS uint32_t*)h.pen;
  if (need_cnt) {
    for (uint32_t i = tid; i < Uc; i += NT) cnt[i] = 0;
    __syncthreads();
    for (uint32_t c0 = h0; c0 < h1; c0 += HTPT * NT) {
#pragma unroll
      for (int q = 0; q < HTPT; ++q) {
        uint32_t t = tk[q];
        const uint32_t i = c0 + q * NT + tid;
        if (!one_pass) t = (i < h1) ? G(a.htok)[i] : EMPTY;
        if (t >= lo && t < hi) {
          const uint32_t r = h.rank(t);
          if (r < U_MAX) __atomic_fetch_add(&cnt[r], hist_weight(a, i), __ATOMIC_RELAXED);
        }
      }
    }
  }
  __syncthreads();
  // penalised logit of every distinct history token: loads first, then math
  for (uint32_t r0 = 0; r0 < Uc; r0 += HTPT * NT) {
    float x[HTPT];
#pragma unroll
    for (int q = 0; q < HTPT; ++q) {
      const uint32_t r = r0 + q * NT + tid;
      x[q] = (r < Uc) ? load_logit<DT>(row, h.tokr[r]) : 0.0f;
    }
#pragma unroll
    for (int q = 0; q < HTPT; ++q) {
      const uint32_t r = r0 + q * NT + tid;
      if (r < Uc) h.pen[r] = penalize(x[q], P, need_cnt ? cnt[r] : 1u);
    }
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// Candidate-threshold histogram
// ---------------------------------------------------------------------------
// Largest fine bin beta such that at least Kc counted elements have bin >=
// beta (0 if fewer are counted).  Counts are lower bounds of the true counts,
// so beta never exceeds the bin of the true Kc-th largest logit.
__device__ __forceinline__ uint32_t compute_beta(LDS const uint32_t* hc, LDS const uint32_t* hf,
                                 uint32_t Kc, int lane) {
  const uint32_t c = hc[63 - lane];
  const uint32_t incl = wave_incl_scan(c);
  const uint64_t m = __ballot(incl >= Kc);
  if (m == 0) return 0;
  const int l = __ffsll((unsigned long long)m) - 1;
  const uint32_t cb = 63u - (uint32_t)l;
  const uint32_t before = __shfl(incl - c, l);
  const uint32_t need = Kc - before;
  const uint32_t f = hf[cb * 64 + 63 - lane];
  const uint32_t fincl = wave_incl_scan(f);
  const uint64_t m2 = __ballot(fincl >= need);
  if (m2 == 0) return 0;
  const int l2 = __ffsll((unsigned long long)m2) - 1;
  return cb * 64u + 63u - (uint32_t)l2;
}

// Smallest float whose key lies in bin `beta` (all finite values for the
// bins below that of -FLT_MAX, which hold only NaN and -inf keys).  For
// finite v: v >= theta_of(beta) exactly when bin(v) >= beta, except that
// -0.0 also passes at beta = bin(+0.0), which only adds a candidate.
__device__ __forceinline__ float theta_of(uint32_t beta) {
  return beta <= 8u ? -3.402823466e+38f : funkey(beta << BIN_SHIFT);
}

// ---------------------------------------------------------------------------
// Geometry
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

struct Raw {
  uint32_t d[16];  // fp32 bits (bf16: 8 dwords of pairs)
  uint32_t mw[4];  // allow-mask words of the lane's 4 runs
};

// The vocabulary index of the lane's value j of the tile at tb: an f32 tile
// is four runs of 256 tokens, the lane holding 4 consecutive tokens of each
// (one 16-byte load per run); a 16-bit tile two runs of 512, the lane holding
// 8 consecutive tokens of each (again one 16-byte load per run).
template <int DT>
__device__ __forceinline__ uint32_t tile_pos(uint32_t tb, int lane, int j) {
  if ((DT & 3) == LLMK_F32)
    return tb + 256u * (uint32_t)(j >> 2) + 4u * (uint32_t)lane + (uint32_t)(j & 3);
  return tb + 512u * (uint32_t)(j >> 3) + 8u * (uint32_t)lane + (uint32_t)(j & 7);
}

// Lane `lane` owns the tile positions tile_pos gives.
template <int DT>
__device__ __forceinline__ void load_tile(const Args& a, const void* row,
                                          const uint32_t* mrow, const Hist& h,
                                          uint32_t t, int lane, Raw& raw) {
  const uint32_t tb = t * TILE;
  (void)h;
  if (tb + TILE <= a.V) {
    if ((DT & 3) == LLMK_F32) {
      const GLB f4v* p = (const GLB f4v*)G((const float*)row + tb) + lane;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const f4v x = __builtin_nontemporal_load(p + 64 * r);
        raw.d[4 * r + 0] = __float_as_uint(x.x);
        raw.d[4 * r + 1] = __float_as_uint(x.y);
        raw.d[4 * r + 2] = __float_as_uint(x.z);
        raw.d[4 * r + 3] = __float_as_uint(x.w);
      }
    } else {
      // two 16-byte loads: tokens 512h + 8 lane .. 512h + 8 lane + 7
      const GLB u4v* p = (const GLB u4v*)G((const uint16_t*)row + tb) + lane;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const u4v x = __builtin_nontemporal_load(p + 64 * hh);
        raw.d[4 * hh + 0] = x.x;
        raw.d[4 * hh + 1] = x.y;
        raw.d[4 * hh + 2] = x.z;
        raw.d[4 * hh + 3] = x.w;
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t e = tile_pos<DT>(tb, lane, j);
      if ((DT & 3) == LLMK_F32) {
        raw.d[j] = e < a.V ? G((const uint32_t*)row)[e] : 0xff800000u;  // -inf past V
      } else {
        // the raw 16-bit value, -inf past V
        const uint32_t hv = e < a.V ? (uint32_t)G((const uint16_t*)row)[e]
                                    : ((DT & 3) == LLMK_BF16 ? 0xff80u : 0xfc00u);
        if ((j & 1) == 0) raw.d[j >> 1] = hv;
        else raw.d[j >> 1] |= hv << 16;
      }
    }
  }
  if (mrow) {
    if ((DT & 3) == LLMK_F32) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t wi = (tb >> 5) + 8u * r + ((uint32_t)lane >> 3);
        raw.mw[r] = (wi < a.mask_words) ? G(mrow)[wi] : 0u;
      }
    } else {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const uint32_t wi = (tb >> 5) + 16u * hh + ((uint32_t)lane >> 2);
        raw.mw[hh] = (wi < a.mask_words) ? G(mrow)[wi] : 0u;
      }
    }
  }
}

template <int DT>
__device__ __forceinline__ void unpack(const Raw& raw, float v[16]) {
  if ((DT & 3) == LLMK_F32) {
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = __uint_as_float(raw.d[j]);
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if ((DT & 3) == LLMK_BF16) {
        v[4 * r + 0] = __uint_as_float(raw.d[2 * r] << 16);
        v[4 * r + 1] = __uint_as_float(raw.d[2 * r] & 0xffff0000u);
        v[4 * r + 2] = __uint_as_float(raw.d[2 * r + 1] << 16);
        v[4 * r + 3] = __uint_as_float(raw.d[2 * r + 1] & 0xffff0000u);
      } else {
        v[4 * r + 0] = cvt16<DT>(raw.d[2 * r] & 0xffffu);
        v[4 * r + 1] = cvt16<DT>(raw.d[2 * r] >> 16);
        v[4 * r + 2] = cvt16<DT>(raw.d[2 * r + 1] & 0xffffu);
        v[4 * r + 3] = cvt16<DT>(raw.d[2 * r + 1] >> 16);
      }
    }
  }
  if (DT & SOFTCAP) {
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = softcap<DT>(v[j]);
  }
}

// ---------------------------------------------------------------------------
// Probabilities and the sequential semantics
// ---------------------------------------------------------------------------
// p of a (penalised, masked) logit v given the temperature, x_max = m and
// the normaliser S: sampler.rs:53-70, with glibc's expf (exp_ref).  S is
// the reference's sequential sum, or 1 on a row that top-k renormalises
// (where S cancels: p is then e itself).
__device__ __forceinline__ float prob_of(float v, float T, float m, float S) {
  const float x = (T != 1.0f) ? v / T : v;
  const float e = (x == NEG_INF) ? 0.0f : exp_ref(x - m);
  return (S > 0.0f) ? e / S : e;
}

__device__ __forceinline__ uint64_t pkey(float p, uint32_t idx) {
  return ((uint64_t)(~__float_as_uint(p)) << 32) | idx;
}

// Synchronisation policies: a whole workgroup (barriers) or one wave (LDS
// traffic of a single wave completes in order; waiting for it suffices).
// excl_scan(keep): this thread's position among the keeping threads of the
// policy (in id order) and their total.
struct BlockSync {
  static constexpr uint32_t N = NT;
  __device__ static __forceinline__ uint32_t id() { return threadIdx.x; }
  __device__ static __forceinline__ void sync() { __syncthreads(); }
  __device__ static __forceinline__ uint32_t excl_scan(bool keep, LDS uint32_t* red,
                                                       uint32_t& total) {
    return block_excl_scan(keep ? 1u : 0u, red, total);
  }
};
struct WaveSync {
  static constexpr uint32_t N = WAVE;
  __device__ static __forceinline__ uint32_t id() { return threadIdx.x & 63u; }
  __device__ static __forceinline__ void sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS ops done
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  __device__ static __forceinline__ uint32_t excl_scan(bool keep, LDS uint32_t*,
                                                       uint32_t& total) {
    const uint64_t mk = __ballot(keep);
    total = (uint32_t)__popcll(mk);
    return lanes_below(mk);
  }
};

// A list sorted by (p desc, idx asc) holding the probabilities as first
// computed; renormalisations (sampler.rs:84-87, :104-109) are recorded as a
// chain of divisors and applied on every read, fl(fl(p/s1)/s2), exactly as
// the reference's in-place divisions, so the list itself is never rewritten.
struct Chain {
  float d0, d1, d2;
  int n;
  __device__ __forceinline__ float apply(float x) const {
    if (n > 0) x = x / d0;
    if (n > 1) x = x / d1;
    if (n > 2) x = x / d2;
    return x;
  }
  __device__ __forceinline__ void push(float s) {
    if (n == 0) d0 = s;
    else if (n == 1) d1 = s;
    else d2 = s;
    ++n;
  }
};
// p and idx are generic pointers (LDS or global memory): one type, so the
// semantics below are compiled once.
struct List {
  const float* p;
  const uint32_t* idx;
  Chain c;
  float* wp;  // p, writable (an LDS list): renormalisations rewrite it
  __device__ float raw(uint32_t i) const { return p[i]; }
  __device__ float get(uint32_t i) const { return c.apply(p[i]); }
  __device__ uint32_t id(uint32_t i) const { return idx[i]; }
};
template <class T>
__device__ __forceinline__ const T* flat(LDS const T* x) {
  return (const T*)x;
}
template <class T>
__device__ __forceinline__ const T* flat(const GLB T* x) {
  return (const T*)x;
}

__device__ __forceinline__ float rl(float x, uint32_t j) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), (int)j));
}

// Increments of the running sum, in units of the binade's quantum, from an
// even (a0) and from an odd (a1) running sum.
struct Par {
  uint32_t a0, a1;
};
// f, then g
__device__ __forceinline__ Par par_then(Par f, Par g) {
  return Par{f.a0 + ((f.a0 & 1u) ? g.a1 : g.a0), f.a1 + ((f.a1 & 1u) ? g.a0 : g.a1)};
}

// The sequential f32 running sums ((p_0 + p_1) + p_2) + ... of list[0..n),
// exactly, computed by wave 0 a window of 512 entries at a time (8
// consecutive entries per lane).  While the running sum c lies in the binade
// [2^e, 2^(e+1)) (e >= -126 also covers the subnormals), c is a multiple of
// q = 2^(e-23), c/q < 2^24, and fl(c + p) is c + q*r with r the nearest
// integer to p/q, a tie going to the even sum: r depends on p alone except
// for a tie, where it depends on the parity of c/q.  So every entry is a
// pair of integer increments (from an even, from an odd sum), and a wave scan
// of the pairs gives every running sum of the binade exactly.  The first
// addition whose result would reach 2^(e+1) is done as one f32 addition and
// the scan resumes after it (a sum of probabilities crosses a few tens of
// binades at most).  Every thread calls it.
// mode 0: sum of all n.  mode 1: stop at the first j with cum >= thr.
// mode 2: stop at the first j with thr <= cum (the draw's `r <= cumulative`).
// Returns the stop index (n if none) and the running sum including it (the
// total if none).  sh: 2 words; z: 128 words.
// Every lane forms its own prefix: lane l of c0 receives ((p_0 + p_1) + ...)
// + p_l and lane l of c1 the prefix through entry 64 + l -- the same f32
// additions in the same order as one sequential sum.  z holds 64 zeros before
// each half of the entries; lane l reads z[1 + l + t] at step t = 0..63, so it
// adds 63 - l zeros (+0.0 + +0.0 stays +0.0) and then p_0..p_l.  All 64 reads
// are issued before the adds and there is no branch: two operations per step.
// Lanes at or past m hold junk.
__device__ __forceinline__ float prefix_half(LDS const float* zb, float c) {
  float x[64];
#pragma unroll
  for (uint32_t t = 0; t < 64u; ++t) x[t] = zb[t];
#pragma unroll
  for (uint32_t t = 0; t < 64u; ++t) c = c + x[t];
  return c;
}
// prefix_half with sixteen reads in flight at a time (fewer registers)
__device__ __forceinline__ float prefix_half16(LDS const float* zb, float c) {
#pragma unroll
  for (uint32_t t0 = 0; t0 < 64u; t0 += 16u) {
    float x[16];
#pragma unroll
    for (uint32_t t = 0; t < 16u; ++t) x[t] = zb[t0 + t];
#pragma unroll
    for (uint32_t t = 0; t < 16u; ++t) c = c + x[t];
  }
  return c;
}
// Exclusive scan of the pairs over the wave (DPP row shifts and row
// broadcasts; shifted-in lanes read (0, 0), the identity).
template <int CTRL, int RM, bool BC>
__device__ __forceinline__ Par dpp_par(Par x) {
  return Par{dppu<CTRL, RM, BC>(0u, x.a0), dppu<CTRL, RM, BC>(0u, x.a1)};
}
__device__ __forceinline__ Par wave_par_excl(Par x) {
  x = par_then(dpp_par<0x111, 0xf, true>(x), x);
  x = par_then(dpp_par<0x112, 0xf, true>(x), x);
  x = par_then(dpp_par<0x114, 0xf, true>(x), x);
  x = par_then(dpp_par<0x118, 0xf, true>(x), x);
  x = par_then(dpp_par<0x142, 0xa, false>(x), x);
  x = par_then(dpp_par<0x143, 0xc, false>(x), x);
  return dpp_par<0x138, 0xf, true>(x);  // wave_shr:1
}
template <int Q>
__device__ __forceinline__ float pickf(const float (&x)[Q], uint32_t k) {
  float r = x[0];
#pragma unroll
  for (int q = 1; q < Q; ++q) r = (k == (uint32_t)q) ? x[q] : r;
  return r;
}
template <class L>
__device__ __forceinline__ uint32_t seq_scan(const L& list, uint32_t n, int mode, float thr,
                                             float& cum_out, LDS uint32_t* sh, LDS float* z) {
  if (threadIdx.x < WAVE) {
    constexpr uint32_t Q = 8, W = Q * WAVE;
    constexpr uint32_t TOP = 1u << 24;
    const uint32_t lane = threadIdx.x, l0 = Q * lane;
    const bool stops = mode != 0;
    uint32_t stop = n;
    float c = 0.0f;
    uint32_t j0 = 0;
    if (n > 0 && stops && thr <= 0.0f) {  // the first running sum already meets it
      stop = 0;
      c = 0.0f + list.get(0);
    } else if (n > 0) {
      // the first 256 entries, where the sum crosses binades often, 64 at a
      // time: every lane forms its own running sum (prefix_half16 from c:
      // 63 - lane zeros, which leave c as it is, then p_base .. p_base+lane,
      // the same f32 additions in the same order)
      const uint32_t hn = umin(n, 4u * WAVE);
      while (j0 < hn) {
        const uint32_t h = umin(hn - j0, (uint32_t)WAVE);
        z[lane] = 0.0f;
        z[WAVE + lane] = lane < h ? list.get(j0 + lane) : 0.0f;
        WaveSync::sync();
        const float cl = prefix_half16(z + 1 + lane, c);
        WaveSync::sync();
        const uint64_t hit = stops ? __ballot(lane < h && cl >= thr) : 0ull;
        if (hit) {
          const uint32_t js = (uint32_t)__ffsll((unsigned long long)hit) - 1;
          stop = j0 + js;
          c = rl(cl, js);
          break;
        }
        c = rl(cl, h - 1);
        j0 += h;
      }
    }
    // the raw entries of the window at jj (the divisor chain is applied when
    // it is scanned); the next window's are requested before a window is
    // scanned, so that a list in global memory is not waited for window by
    // window
    float pr[Q];
    auto fetch = [&](uint32_t jj) __attribute__((always_inline)) {
#pragma unroll
      for (uint32_t q = 0; q < Q; ++q) pr[q] = jj + l0 + q < n ? list.raw(jj + l0 + q) : 0.0f;
    };
    if (j0 < n && stop == n) fetch(j0);
    for (uint32_t j = j0; j < n && stop == n; j += W) {
      const uint32_t lim = umin(n - j, W);
      float p[Q];
#pragma unroll
      for (uint32_t q = 0; q < Q; ++q) p[q] = (l0 + q < lim) ? list.c.apply(pr[q]) : 0.0f;
      if (j + W < n) fetch(j + W);
      uint32_t s = 0;  // window entries before s are summed
      while (s < lim) {
        if (c == 0.0f) {
          // 0 + p is exact: the first nonzero entry starts the sum (zeros
          // leave it 0, below thr > 0)
          uint32_t fz = EMPTY;
#pragma unroll
          for (int q = (int)Q - 1; q >= 0; --q)
            if (l0 + q >= s && l0 + q < lim && p[q] != 0.0f) fz = l0 + q;
          fz = wave_min_u32(fz);
          if (fz == EMPTY) {
            s = lim;
            break;
          }
          c = 0.0f + rl(pickf(p, fz % Q), fz / Q);
          s = fz + 1;
          if (stops && c >= thr) {
            stop = j + fz;
            break;
          }
          continue;
        }
        const uint32_t cb = __float_as_uint(c);
        const int e = (int)umax((cb >> 23) & 255u, 1u) - 127;
        const uint32_t C = (uint32_t)__builtin_ldexpf(c, 23 - e);
        uint32_t r[Q], tie = 0;  // increments; ties: the value from an even sum differs
#pragma unroll
        for (uint32_t q = 0; q < Q; ++q) {
          const float x = __builtin_ldexpf(p[q], 23 - e);  // exact, < 2^24
          const float k = __builtin_floorf(x);
          const float fr = x - k;
          const uint32_t ki = (uint32_t)k;
          const bool live = l0 + q >= s && l0 + q < lim;
          r[q] = !live ? 0u : (fr > 0.5f ? ki + 1u : ki);
          if (live && fr == 0.5f) tie |= 1u << q;
        }
        // this lane's increments from an even and from an odd sum (a tie
        // adds k or k + 1, whichever makes the sum even)
        uint32_t s0 = 0, s1 = 1;
#pragma unroll
        for (uint32_t q = 0; q < Q; ++q) {
          const uint32_t t = (tie >> q) & 1u;
          s0 += r[q] + (t & ((s0 ^ r[q]) & 1u));
          s1 += r[q] + (t & ((s1 ^ r[q]) & 1u));
        }
        const Par ex = wave_par_excl(Par{s0, s1 - 1u});
        uint32_t cur = C + ((C & 1u) ? ex.a1 : ex.a0);
        // the lane's first event (crossing or stop) with the sum before (a
        // crossing) or at (a stop) it, and the sum at the window's last entry
        uint32_t ev = EMPTY, evv = 0, endv = 0, evx = 0;
#pragma unroll
        for (uint32_t q = 0; q < Q; ++q) {
          const uint32_t t = (tie >> q) & 1u;
          const uint32_t nx = cur + r[q] + (t & ((cur ^ r[q]) & 1u));
          if (ev == EMPTY && l0 + q >= s && l0 + q < lim) {
            if (nx >= TOP) {
              ev = l0 + q;
              evx = 1;
              evv = cur;
            } else if (stops && __builtin_ldexpf((float)nx, e - 23) >= thr) {
              ev = l0 + q;
              evv = nx;
            }
          }
          if (l0 + q == lim - 1) endv = nx;
          cur = nx;
        }
        const uint32_t evm = wave_min_u32(ev);
        if (evm == EMPTY) {
          const uint32_t v = (uint32_t)__builtin_amdgcn_readlane((int)endv, (int)((lim - 1) / Q));
          c = __builtin_ldexpf((float)v, e - 23);
          s = lim;
          break;
        }
        const int ol = (int)(evm / Q);
        const float v =
            __builtin_ldexpf((float)(uint32_t)__builtin_amdgcn_readlane((int)evv, ol), e - 23);
        if (!__builtin_amdgcn_readlane((int)evx, ol)) {
          stop = j + evm;
          c = v;
          break;
        }
        // the addition that leaves the binade, as one f32 addition
        c = v + rl(pickf(p, evm % Q), (uint32_t)ol);
        s = evm + 1;
        if (stops && c >= thr) {
          stop = j + evm;
          break;
        }
      }
    }
    if (lane == 0) {
      sh[0] = stop;
      sh[1] = __float_as_uint(c);
    }
  }
  __syncthreads();
  const uint32_t stop = sh[0];
  cum_out = __uint_as_float(sh[1]);
  __syncthreads();
  return stop;
}

// The renormalisation p /= s of the first len entries (sampler.rs:84-87,
// :104-109): rewritten in place for a writable list (every thread calls
// it), else recorded in the divisor chain.
__device__ __forceinline__ void div_all(List& list, float s, uint32_t len) {
  if (!(s > 0.0f)) return;
  if (list.wp) {
    for (uint32_t i = threadIdx.x; i < len; i += NT) list.wp[i] = list.wp[i] / s;
    __syncthreads();
  } else {
    list.c.push(s);
  }
}

// First i < n with list[i] < thr (strict) or <= thr, n if none; the list is
// sorted descending, so the predicate is monotone: one probe per thread
// finds the block of n/NT entries holding the first hit, then the block is
// searched.  n <= NT * NT.  sh: 1 word.
__device__ __forceinline__ uint32_t first_below(const List& list, uint32_t n, float thr,
                                                bool strict,
                                LDS uint32_t* sh) {
  const uint32_t tid = threadIdx.x;
  auto hit = [&](uint32_t i) {
    const float v = list.get(i);
    return strict ? v < thr : v <= thr;
  };
  const uint32_t step = (n + NT - 1) / NT;
  if (tid == 0) sh[0] = EMPTY;
  __syncthreads();
  const uint32_t lo = tid * step;
  if (lo < n && hit(umin(lo + step, n) - 1)) __atomic_fetch_min(&sh[0], tid, __ATOMIC_RELAXED);
  __syncthreads();
  const uint32_t kb = sh[0];
  __syncthreads();
  if (kb == EMPTY) return n;
  if (tid == 0) sh[0] = EMPTY;
  __syncthreads();
  const uint32_t b0 = kb * step;
  if (tid < step && b0 + tid < n && hit(b0 + tid))
    __atomic_fetch_min(&sh[0], b0 + tid, __ATOMIC_RELAXED);
  __syncthreads();
  const uint32_t r = sh[0];
  __syncthreads();
  return r;
}

// Lists at least this long are scanned by the whole workgroup
// (block_list_scan), shorter ones by wave 0 (seq_scan); only the slow path's
// lists get that long (the candidate path keeps at most SORT_CAP).
constexpr uint32_t BLOCK_SCAN_MIN = 4096;
__device__ __attribute__((noinline)) u2v block_list_scan(List list, uint32_t n, int mode,
                                                        float thr, LDS uint32_t* sc);

// min-p / top-k / top-p / draw (sampler.rs:77-124 + min-p) over a sorted list
// of full_len entries whose first E are exact; every entry past E has
// p <= ptail.  Every thread of the workgroup.  Returns false if an entry
// beyond E would be needed.  The four steps share one running-sum call.
template <bool LONG>
__device__ __forceinline__ bool run_semantics(const RowP& P, float u, uint32_t E,
                                              uint32_t full_len, float ptail, List& list,
                                              LDS uint32_t* sh, LDS float* z,
                                              uint32_t& tok_out, uint32_t& len_out) {
  uint32_t len = full_len;
  bool trunc = E < full_len;
  for (int step = 0; step < 4; ++step) {
    uint32_t n;
    int mode = 0;
    float thr = 0.0f;
    if (step == 0) {
      // ---- min-p (extension): keep p >= min_p * p_max, renormalise if it cuts
      if (!(P.min_p > 0.0f)) continue;
      if (E == 0) return false;
      const float t = P.min_p * list.get(0);
      const uint32_t lim = E < len ? E : len;
      uint32_t cut = first_below(list, lim, t, true, sh);
      if (cut == lim) cut = EMPTY;
      // every entry past E is below the threshold: the cut is at E
      if (cut == EMPTY && trunc && ptail < t) cut = E;
      if (cut == EMPTY) {
        if (trunc) return false;
        continue;
      }
      if (cut >= len) continue;
      len = cut;
      trunc = false;
      n = len;
    } else if (step == 1) {
      // ---- top-k, sampler.rs:80-89
      if (!(P.K > 0 && (uint32_t)P.K < len)) continue;
      if ((uint32_t)P.K > E) return false;
      len = (uint32_t)P.K;
      trunc = false;
      n = len;
    } else {
      // ---- top-p, sampler.rs:92-110; the draw, sampler.rs:113-124
      if (step == 2 && !(P.top_p < 1.0f)) continue;
      n = (trunc && E < len) ? E : len;
      mode = step == 2 ? 1 : 2;
      thr = step == 2 ? P.top_p : u;
    }
    float s;
    uint32_t j;
    if (LONG && n >= BLOCK_SCAN_MIN) {
      const u2v r = block_list_scan(list, n, mode, thr, (LDS uint32_t*)z);
      j = r.x;
      s = __uint_as_float(r.y);
    } else {
      j = seq_scan(list, n, mode, thr, s, sh, z);
    }
    if (step == 3) {
      uint32_t tok;
      if (j < n) tok = list.id(j);
      else {
        if (trunc) return false;
        tok = len > 0 ? list.id(len - 1) : 0u;
      }
      tok_out = tok;
      len_out = len;
      return true;
    }
    if (step == 2) {
      if (j == n && trunc) return false;
      // the renormalisation sum over the kept prefix is the same sequential
      // sum as the cumulative at the cut
      len = (j < n) ? j + 1 : len;
      trunc = false;
    }
    div_all(list, s, len);
  }
  return false;
}

__device__ __forceinline__ void write_outputs(const Args& a, uint32_t b, uint32_t tok,
                                              uint32_t len, const List& list, float m,
                                              float S) {
  if (threadIdx.x == 0) {
    G(a.out_tok)[b] = tok;
    if (a.out_cnt) G(a.out_cnt)[b] = len;
    if (a.cut)
      G(a.cut)[b] = u4v{(len > 0 && len < a.V) ? list.id(len - 1) : 0u, len,
                        __float_as_uint(m), __float_as_uint(S)};
  }
  if (a.out_cap) {
    const uint32_t n = len < a.out_cap ? len : a.out_cap;
    for (uint32_t j = threadIdx.x; j < n; j += NT) {
      if (a.out_ids) G(a.out_ids)[(uint64_t)b * a.out_cap + j] = list.id(j);
      if (a.out_probs) G(a.out_probs)[(uint64_t)b * a.out_cap + j] = list.get(j);
    }
  }
}

// ---------------------------------------------------------------------------
// min-p / top-k / top-p / draw for a sorted list of at most 128 entries held
// in registers of one wave: lane j holds entries j (p0, i0) and 64 + j (p1,
// i1).  The same sequential f32 sums and divisions as run_semantics, in the
// same order; the running sums are wave-uniform, each step reading one entry
// with v_readlane.  Returns false if an entry beyond E = n would be needed.
// ---------------------------------------------------------------------------
// z: 256 LDS words owned by the calling wave; 1 <= m <= 128.
__device__ __forceinline__ void prefix_regs(float p0, float p1, uint32_t m, int lane,
                                            LDS float* z, float& c0, float& c1) {
  z[lane] = 0.0f;
  z[64 + lane] = p0;
  z[128 + lane] = 0.0f;
  z[192 + lane] = p1;
  WaveSync::sync();
  c0 = prefix_half(z + 1 + lane, 0.0f);
  c1 = 0.0f;
  if (m > 64u) c1 = prefix_half(z + 129 + lane, rl(c0, 63));
  WaveSync::sync();  // z is rewritten by the next call
}
// ((p_0 + p_1) + ...) + p_{m-1}
__device__ __forceinline__ float seq_sum_regs(float p0, float p1, uint32_t m, int lane,
                                              LDS float* z) {
  if (m == 0) return 0.0f;
  float c0, c1;
  prefix_regs(p0, p1, m, lane, z, c0, c1);
  return m <= 64 ? rl(c0, m - 1) : rl(c1, m - 65);
}
// First j < m whose running sum meets the condition (mode 1: cum >= thr,
// mode 2: thr <= cum), m if none; cum_out: the running sum there (or the
// total).
__device__ __forceinline__ uint32_t seq_find_regs(float p0, float p1, uint32_t m, int mode,
                                                  float thr, int lane, LDS float* z,
                                                  float& cum_out) {
  if (m == 0) {
    cum_out = 0.0f;
    return 0;
  }
  float c0, c1;
  prefix_regs(p0, p1, m, lane, z, c0, c1);
  auto meets = [&](float x) { return mode == 1 ? x >= thr : thr <= x; };
  const uint64_t m0 = __ballot((uint32_t)lane < m && meets(c0));
  const uint64_t m1 = __ballot((uint32_t)lane + 64 < m && meets(c1));
  uint32_t j = m;
  if (m0) j = (uint32_t)__ffsll((unsigned long long)m0) - 1;
  else if (m1) j = 64u + (uint32_t)__ffsll((unsigned long long)m1) - 1;
  const uint32_t jc = j < m ? j : m - 1;
  cum_out = jc < 64 ? rl(c0, jc) : rl(c1, jc - 64);
  return j;
}

// Index of kept entry len - 1 of a register list of n (wave-uniform), 0 when
// it is not held (len 0, or every entry kept).
__device__ __forceinline__ uint32_t cut_id(uint32_t len, uint32_t n, uint32_t i0, uint32_t i1) {
  const uint32_t lc = (len > 0 && len <= n) ? len - 1 : 0u;
  const uint32_t v = lc < 64 ? (uint32_t)__builtin_amdgcn_readlane((int)i0, (int)lc)
                             : (uint32_t)__builtin_amdgcn_readlane((int)i1, (int)(lc - 64));
  return (len > 0 && len <= n) ? v : 0u;
}

// ---------------------------------------------------------------------------
// The rounding band of S = 1 on rows that top-k renormalises
// ---------------------------------------------------------------------------
// Such a row is sampled with S = 1 (p = e): the reference divides by its
// sequential sum S first (sampler.rs:66-71) and by a renormalising sum before
// any later step reads a probability (min-p's cut, then top-k, :83-88), so S
// cancels in exact arithmetic.  band_certain_wave proves from the sorted e
// alone that every decision (min-p cut, top-k set and order, top-p cut at
// :97, the draw at :118) is the reference's for any S it can hold; a row it
// cannot prove is sampled again with the reference's own S.  The bound: p
// known to relative R (2^-24 for fl(e / S)); a sequential sum rounds each
// partial sum by at most half an ulp of it (u times the value while the
// scale is S's, the binade's half ulp once normalised); a renormalisation
// divides by a sum known to relative sigma and rounds once more:
// R' = (R + sigma + u)(1 + 2^-10), the factor covering second-order terms.
// A decision is certain when its exact value (sums of the e in double)
// lies outside its bound; order is certain unless two entries within 2^-20
// relative have their indices inverted (fl(e_a/S) == fl(e_b/S) ties go by
// index); entries below 2^-100 (p could be subnormal) are never certain.
// The doubles are summed in one fixed order, which the CPU oracle follows:
// a wave's DPP scan within 64 entries (row_shr 1, 2, 4, 8 within rows of 16,
// then row_bcast 15 and 31), then the chunk's carry.  One wave; acc(j) =
// (e bits, index) of entry j < E; entries past E are <= ptail.
constexpr double BAND_U = 0x1p-24;
constexpr double BAND_F = 1.0 + 0x1p-10;
constexpr double BAND_SL = 0x1p-36;
constexpr double BAND_CLOSE = 1.0 + 0x1p-20;
// half an ulp of a float of magnitude x in (0, 2): 2^(floor(log2 x) - 24)
__device__ __forceinline__ double band_hu(double x) {
  if (!(x > 0.0)) return 0.0;
  const uint64_t ex = ((uint64_t)__double_as_longlong(x) >> 52) & 0x7ffu;
  return __longlong_as_double((long long)((ex - 24u) << 52));
}
template <int CTRL, int RM, bool BC>
__device__ __forceinline__ double dppd(double x) {
  const uint64_t b = (uint64_t)__double_as_longlong(x);
  const uint32_t lo = dppu<CTRL, RM, BC>(0u, (uint32_t)b);
  const uint32_t hi = dppu<CTRL, RM, BC>(0u, (uint32_t)(b >> 32));
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
// inclusive prefix over the wave (lanes outside a step's reach add +0)
__device__ __forceinline__ double wave_prefix_d(double x) {
  x = x + dppd<0x111, 0xf, true>(x);
  x = x + dppd<0x112, 0xf, true>(x);
  x = x + dppd<0x114, 0xf, true>(x);
  x = x + dppd<0x118, 0xf, true>(x);
  x = x + dppd<0x142, 0xa, false>(x);
  x = x + dppd<0x143, 0xc, false>(x);
  return x;
}
__device__ __forceinline__ double readlane_d(double x, int l) {
  const uint64_t b = (uint64_t)__double_as_longlong(x);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), l);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
template <class ACC>
struct BandList {
  ACC acc;
  uint32_t E;
  __device__ __forceinline__ double e(uint32_t j) const {
    return j < E ? (double)__uint_as_float(acc(j).x) : 0.0;
  }
  // P_{n-1} (prefix of e over [0, n)) and sum_{1 <= j < n} P_j
  __device__ __forceinline__ void sums(uint32_t n, int lane, double& ptot, double& qtot) const {
    double cp = 0.0, cq = 0.0;
    for (uint32_t c0 = 0; c0 < n; c0 += WAVE) {
      const uint32_t j = c0 + (uint32_t)lane;
      const double Pj = wave_prefix_d(j < n ? e(j) : 0.0) + cp;
      const double Qj = wave_prefix_d((j < n && j >= 1) ? Pj : 0.0) + cq;
      if (c0 + WAVE >= n) {
        ptot = readlane_d(Pj, (int)((n - 1) & 63u));
        qtot = readlane_d(Qj, (int)((n - 1) & 63u));
      } else {
        cp = readlane_d(Pj, 63);
        cq = readlane_d(Qj, 63);
      }
    }
  }
  // The first j < n whose cumulative may reach thr (C_j + B_j >= thr), n if
  // none; certain: the reference's cumulative surely reaches it there and
  // not before.  C_j = P_j (1 / tot), B_j = R C_j + sum_{1<=i<=j} hu(C_i (1 +
  // R) F) + SL C_j.  bj, pj: B_j and P_j there (at n - 1 when none).
  __device__ __forceinline__ uint32_t find(uint32_t n, double tot, double R, double thr,
                                           int lane, bool& certain, double& bj,
                                           double& pj) const {
    const double rt = 1.0 / tot;
    double cp = 0.0, ch = 0.0;
    for (uint32_t c0 = 0; c0 < n; c0 += WAVE) {
      const uint32_t j = c0 + (uint32_t)lane;
      const double Pj = wave_prefix_d(j < n ? e(j) : 0.0) + cp;
      const double C = Pj * rt;
      const double hj = (j < n && j >= 1) ? band_hu(C * (1.0 + R) * BAND_F) : 0.0;
      const double Hj = wave_prefix_d(hj) + ch;
      const double b = R * C + Hj + BAND_SL * C;
      const uint64_t hit = __ballot(j < n && C + b >= thr);
      if (hit) {
        const int l = __ffsll((unsigned long long)hit) - 1;
        certain = __builtin_amdgcn_readlane((int)(C - b >= thr), l) != 0;
        bj = readlane_d(b, l);
        pj = readlane_d(Pj, l);
        return c0 + (uint32_t)l;
      }
      if (c0 + WAVE >= n) {
        bj = readlane_d(b, (int)((n - 1) & 63u));
        pj = readlane_d(Pj, (int)((n - 1) & 63u));
      } else {
        cp = readlane_d(Pj, 63);
        ch = readlane_d(Hj, 63);
      }
    }
    certain = true;
    return n;
  }
};
// sorted (p desc, idx asc) keys
struct KeyAcc {
  LDS const uint64_t* k;
  __device__ __forceinline__ u2v operator()(uint32_t j) const {
    const uint64_t x = k[j];
    return u2v{~(uint32_t)(x >> 32), (uint32_t)x};
  }
};
// sorted p and index arrays (LDS or global)
template <class PF, class PI>
struct ArrAcc {
  PF p;
  PI i;
  __device__ __forceinline__ u2v operator()(uint32_t j) const {
    return u2v{__float_as_uint(p[j]), i[j]};
  }
};
template <class ACC>
__device__ __noinline__ bool band_certain_wave(ACC acc, uint32_t E, uint32_t full,
                                               float ptail, float min_p, int32_t K,
                                               float top_p, float u) {
  const int lane = (int)(threadIdx.x & 63u);
  const BandList<ACC> L{acc, E};
  uint32_t len = full;
  double R = BAND_U;
  bool normalised = false;
  // entries whose p = e / S could be subnormal
  const uint32_t lim = (K > 0 && (uint32_t)K + 1u < E) ? (uint32_t)K + 1u : E;
  for (uint32_t c0 = 0; c0 < lim; c0 += WAVE) {
    const uint32_t j = c0 + (uint32_t)lane;
    const float x = j < lim ? __uint_as_float(acc(j).x) : 0.0f;
    if (__ballot(x > 0.0f && x < 0x1p-100f)) return false;
  }
  double ptot = 0.0, qtot = 0.0;
  auto renormalise = [&](uint32_t n) {
    L.sums(n, lane, ptot, qtot);
    const double sg = R + BAND_U * (1.0 + R) * BAND_F * (qtot / ptot);
    R = (R + sg + BAND_U) * BAND_F;
    normalised = true;
  };
  // min-p: kept iff fl(e/S) >= fl(min_p fl(1/S)) (e_0 = 1, the maximum);
  // certain outside min_p (1 -+ 2^-21)
  if (min_p > 0.0f) {
    if (min_p < 0x1p-100f || E == 0) return false;
    const double hi = (double)min_p * (1.0 + 0x1p-21);
    const double lo = (double)min_p * (1.0 - 0x1p-21);
    const uint32_t n = E < len ? E : len;
    uint32_t cut = EMPTY;
    for (uint32_t c0 = 0; c0 < n; c0 += WAVE) {
      const uint32_t j = c0 + (uint32_t)lane;
      const uint64_t hit = __ballot(j < n && L.e(j) < hi);
      if (hit) {
        cut = c0 + (uint32_t)(__ffsll((unsigned long long)hit) - 1);
        break;
      }
    }
    if (cut != EMPTY) {
      if (L.e(cut) >= lo) return false;
    } else if (E < len) {
      if ((double)ptail >= lo) return false;
      cut = E;
    }
    if (cut != EMPTY && cut < len) {
      len = cut;
      if (len == 0) return false;
      renormalise(len);
      if (!(ptot > 0.0)) return false;
    }
  }
  // top-k: the first K in (p desc, idx asc) order; no pair whose order could
  // change, across the boundary included (an unknown entry K close to the
  // last kept one could be either side of it)
  uint32_t np;
  if (K > 0 && (uint32_t)K < len) {
    if ((uint32_t)K > E) return false;
    if ((uint32_t)K == E && L.e(K - 1) < (double)ptail * BAND_CLOSE) return false;
    np = (uint32_t)K < E ? (uint32_t)K + 1u : (uint32_t)K;
  } else {
    np = E < len ? E : len;
  }
  for (uint32_t c0 = 0; c0 + 1 < np; c0 += WAVE) {
    const uint32_t j = c0 + (uint32_t)lane;
    bool bad = false;
    if (j + 1 < np) {
      const u2v x0 = acc(j), x1 = acc(j + 1);
      bad = (double)__uint_as_float(x0.x) < (double)__uint_as_float(x1.x) * BAND_CLOSE &&
            x0.y > x1.y;
    }
    if (__ballot(bad)) return false;
  }
  if (K > 0 && (uint32_t)K < len) {
    len = (uint32_t)K;
    renormalise(len);
    if (!(ptot > 0.0)) return false;
  }
  if (!normalised || len > E) return false;
  // top-p: the first cumulative >= top_p, then the renormalisation by that
  // same cumulative
  if (top_p < 1.0f) {
    bool cert;
    double b, pc;
    const uint32_t j = L.find(len, ptot, R, (double)top_p, lane, cert, b, pc);
    if (!cert) return false;
    const double sp = b / (pc * (1.0 / ptot));
    R = (R + sp + BAND_U) * BAND_F;
    len = j < len ? j + 1 : len;
    ptot = pc;
  }
  // the draw: the first cumulative >= u, else the last
  bool cert;
  double b, pc;
  (void)L.find(len, ptot, R, (double)u, lane, cert, b, pc);
  return cert;
}

__device__ __forceinline__ bool semantics_regs(const RowP& P, float u, uint32_t n,
                                               uint32_t full_len, float ptail, float& p0,
                                               float& p1,
                                               uint32_t i0, uint32_t i1, int lane,
                                               LDS float* z, uint32_t& tok_out,
                                               uint32_t& len_out) {
  const uint32_t E = n;
  uint32_t len = full_len;
  bool trunc = E < full_len;
  auto divide = [&](float s) {
    if (s > 0.0f) {
      p0 = p0 / s;
      p1 = p1 / s;
    }
  };
  // ---- min-p (extension): keep p >= min_p * p_max, renormalise if it cuts
  if (P.min_p > 0.0f) {
    if (E == 0) return false;
    const float thr = P.min_p * rl(p0, 0);
    const uint32_t lim = E < len ? E : len;
    const uint64_t c0 = __ballot((uint32_t)lane < lim && p0 < thr);
    const uint64_t c1 = __ballot((uint32_t)lane + 64 < lim && p1 < thr);
    uint32_t cut = EMPTY;
    if (c0) cut = (uint32_t)__ffsll((unsigned long long)c0) - 1;
    else if (c1) cut = 64u + (uint32_t)__ffsll((unsigned long long)c1) - 1;
    // every entry past E is below the threshold: the cut is at E
    if (cut == EMPTY && trunc && ptail < thr) cut = E;
    if (cut == EMPTY) {
      if (trunc) return false;
    } else if (cut < len) {
      len = cut;
      trunc = false;
      divide(seq_sum_regs(p0, p1, len, lane, z));
    }
  }
  // ---- top-k, sampler.rs:80-89
  if (P.K > 0 && (uint32_t)P.K < len) {
    if ((uint32_t)P.K > E) return false;
    len = (uint32_t)P.K;
    trunc = false;
    divide(seq_sum_regs(p0, p1, len, lane, z));
  }
  // ---- top-p, sampler.rs:92-110
  if (P.top_p < 1.0f) {
    const uint32_t lim = (trunc && E < len) ? E : len;
    float s;
    const uint32_t j = seq_find_regs(p0, p1, lim, 1, P.top_p, lane, z, s);
    if (j == lim && trunc) return false;
    len = (j < lim) ? j + 1 : len;
    trunc = false;
    divide(s);
  }
  // ---- draw, sampler.rs:113-124
  const uint32_t lim = (trunc && E < len) ? E : len;
  float s;
  const uint32_t j = seq_find_regs(p0, p1, lim, 2, u, lane, z, s);
  uint32_t tok;
  if (j < lim) tok = j < 64 ? (uint32_t)__builtin_amdgcn_readlane((int)i0, (int)j)
                            : (uint32_t)__builtin_amdgcn_readlane((int)i1, (int)(j - 64));
  else {
    if (trunc) return false;
    const uint32_t l1 = len - 1;
    tok = len == 0 ? 0u
                   : (l1 < 64 ? (uint32_t)__builtin_amdgcn_readlane((int)i0, (int)l1)
                              : (uint32_t)__builtin_amdgcn_readlane((int)i1, (int)(l1 - 64)));
  }
  tok_out = tok;
  len_out = len;
  return true;
}

// ---------------------------------------------------------------------------
// Shared-memory layouts (in 32-bit words)
// ---------------------------------------------------------------------------
enum : uint32_t {
  M_BETA = 0, M_CCOUNT = 1, M_FLAGS = 2, M_LAST = 3, M_NEXT = 4,
  M_GSYNC = 5,  // arrivals of the token waves' group barrier
  M_NMISC = 16
};

__host__ __device__ inline size_t stream_lds_words(uint32_t tps) {
  return 64 + M_NMISC + NBINS + 64 + hist_lds_words(tps * 32) + NW;
}
__host__ __device__ inline size_t finalize_lds_words() {
  // slots (2 x MAX_SLOTS) + keys + sorted keys (2 x SORT_CAP u64) + p + idx
  // + scratch + segment table + reductions + block sums
  return 2 * MAX_SLOTS + 4 * SORT_CAP + 2 * SORT_CAP + 128 + MAX_SEG + 16 + 64 + 2 * MAX_SLOTS / 64;
}
__host__ __device__ inline size_t slow_lds_words(uint32_t V) {
  return 128 + 256 + NW * 256 + SLOW_BINS + hist_lds_words((V + 31) / 32);
}

// ---------------------------------------------------------------------------
// The reference's softmax normaliser, exactly (sampler.rs:56-66)
// ---------------------------------------------------------------------------
// Sixteen consecutive logits of a row from e0 (a multiple of 16), as f32;
// positions past V read -inf.
template <int DT>
__device__ __forceinline__ void load16(const void* row, uint32_t e0, uint32_t V, float x[16]) {
  if (e0 + 16 <= V) {
    if ((DT & 3) == LLMK_F32) {
      const GLB f4v* r = (const GLB f4v*)((const GLB float*)row + e0);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const f4v a = r[k];
        x[4 * k + 0] = a.x;
        x[4 * k + 1] = a.y;
        x[4 * k + 2] = a.z;
        x[4 * k + 3] = a.w;
      }
    } else {
      const GLB u2v* r = (const GLB u2v*)((const GLB uint16_t*)row + e0);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const u2v a = r[k];
        x[4 * k + 0] = cvt16<DT>(a.x & 0xffffu);
        x[4 * k + 1] = cvt16<DT>(a.x >> 16);
        x[4 * k + 2] = cvt16<DT>(a.y & 0xffffu);
        x[4 * k + 3] = cvt16<DT>(a.y >> 16);
      }
    }
    if (DT & SOFTCAP) {
#pragma unroll
      for (int q = 0; q < 16; ++q) x[q] = softcap<DT>(x[q]);
    }
  } else {
#pragma unroll
    for (int q = 0; q < 16; ++q) x[q] = e0 + q < V ? load_logit<DT>(row, e0 + q) : NEG_INF;
  }
}

// The smallest of the lanes' keys (~0 = none), whose high words (entry
// indices) differ between lanes that hold one: the minimum high word over
// the wave, then its lane's key.  One LDS atomic per wave then suffices
// (after a crossing every later entry of the window also reports one).
__device__ __forceinline__ uint64_t wave_min_key(uint64_t k) {
  const uint32_t hi = wave_min_u32((uint32_t)(k >> 32));
  const uint64_t owner = __ballot(k != ~0ull && (uint32_t)(k >> 32) == hi);
  if (!owner) return ~0ull;
  const int l = __ffsll((unsigned long long)owner) - 1;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)k, l);
  return ((uint64_t)hi << 32) | lo;
}

// Inclusive scan of the pairs over the wave (shifted-in lanes read the
// identity (0, 0)).
__device__ __forceinline__ Par wave_par_incl(Par x) {
  x = par_then(dpp_par<0x111, 0xf, true>(x), x);
  x = par_then(dpp_par<0x112, 0xf, true>(x), x);
  x = par_then(dpp_par<0x114, 0xf, true>(x), x);
  x = par_then(dpp_par<0x118, 0xf, true>(x), x);
  x = par_then(dpp_par<0x142, 0xa, false>(x), x);
  x = par_then(dpp_par<0x143, 0xc, false>(x), x);
  return x;
}

// The sequential f32 sum c = ((c + e_0) + e_1) + ... of one window's
// entries (all >= 0), continued from c and returned, exactly, by the whole
// workgroup.  Thread t holds entries 16t .. 16t+nq-1 (nq 16, or 4 for a wave
// whose window part was compacted; wave-uniform), so entry j = 16t + q of
// the window comes before entry j' exactly when j < j'.  The running-sum
// argument of seq_scan over the block: while c lies in the binade of quantum
// q = 2^(eb-23), each entry adds the integer r = p/q rounded to nearest (a
// tie to the even sum), a pair of increments (from an even, from an odd sum)
// per entry; the pairs of a thread compose in order, the workgroup scans
// them (waves by DPP, then the sixteen wave totals), and the first entry
// whose sum would reach 2^(eb+1) is added as one f32 addition, after which
// the scan resumes.  Entries p/q >= 2^25 are clamped (they cross at once);
// every sum before the first crossing stays below 2^24 + 2^25, so no count
// wraps where it is read.  A zero c takes the first nonzero entry as it is
// (0 + p = p).  A wave whose entries all lie before the resume point adds
// the identity.  Each round's first event goes through one of three LDS
// slots in turn (round it uses slot it % 3 and clears slot (it + 1) % 3,
// read two rounds ago), so a round needs two barriers; `it` carries the
// rotation from call to call, and the slots start cleared
// (exact_normaliser).  sc: 6 + NW*2 words; uniform barriers only.
//
// block_seq_scan<true> also stops at the first entry whose running sum
// reaches thr (stop_at: its index in the window, EMPTY if none) and returns
// that sum: a stop is an event like a crossing, the first event in index
// order taken, and a crossing's sum is compared with thr after its addition.
template <bool STOPS>
__device__ __forceinline__ float block_seq_scan(const float (&e)[16], uint32_t nq, float c,
                                                uint32_t& it, LDS uint32_t* sc, float thr,
                                                uint32_t& stop_at, uint32_t s_start = 0) {
  constexpr uint32_t Q = 16, TOP = 1u << 24;
  stop_at = EMPTY;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wv = tid >> 6;
  LDS uint64_t* ev = (LDS uint64_t*)sc;  // [3]: first event (index << 32 | new sum bits)
  LDS uint32_t* wt = sc + 6;             // [NW][2]: wave totals
  uint32_t s = s_start;                  // entries before s are summed (into c)
  for (;; ++it) {
    LDS uint64_t* slot = ev + it % 3u;
    if (tid == 0) ev[(it + 1) % 3u] = ~0ull;
    // every entry of this wave lies before s
    const bool wave_done = Q * (64u * wv + 63u) + Q - 1u < s;
    if (c == 0.0f) {
      uint64_t best = ~0ull;
      if (!wave_done) {
#pragma unroll
        for (int q = (int)Q - 1; q >= 0; --q) {
          const uint32_t j = Q * tid + (uint32_t)q;
          if ((uint32_t)q < nq && j >= s && e[q] != 0.0f)
            best = ((uint64_t)j << 32) | __float_as_uint(e[q]);
        }
      }
      best = wave_min_key(best);
      if (lane == 0 && best != ~0ull) __atomic_fetch_min(slot, best, __ATOMIC_RELAXED);
      __syncthreads();
      const uint64_t r = *slot;
      if (r == ~0ull) {  // every remaining entry is 0
        ++it;
        return 0.0f;
      }
      c = __uint_as_float((uint32_t)r);
      s = (uint32_t)(r >> 32) + 1u;
      if (STOPS && c >= thr) {
        stop_at = s - 1u;
        ++it;
        return c;
      }
      if (s >= NT * Q) {
        ++it;
        return c;
      }
      continue;
    }
    const uint32_t cb = __float_as_uint(c);
    const int eb = (int)umax((cb >> 23) & 255u, 1u) - 127;
    const uint32_t C = (uint32_t)__builtin_ldexpf(c, 23 - eb);
    uint32_t r[Q], tie = 0;
    Par own{0u, 0u};
    if (!wave_done) {
#pragma unroll
      for (uint32_t q = 0; q < Q; ++q) {
        r[q] = 0u;
        if (q < nq) {
          const float x = __builtin_fminf(__builtin_ldexpf(e[q], 23 - eb), 0x1p25f);  // exact below the clamp
          const float k = __builtin_floorf(x);
          const float fr = x - k;
          const uint32_t ki = (uint32_t)k;
          const bool live = Q * tid + q >= s;
          r[q] = !live ? 0u : (fr > 0.5f ? ki + 1u : ki);
          if (live && fr == 0.5f) tie |= 1u << q;
        }
      }
      uint32_t s0 = 0, s1 = 1;
#pragma unroll
      for (uint32_t q = 0; q < Q; ++q) {
        if (q < nq) {
          const uint32_t t = (tie >> q) & 1u;
          s0 += r[q] + (t & ((s0 ^ r[q]) & 1u));
          s1 += r[q] + (t & ((s1 ^ r[q]) & 1u));
        }
      }
      own = Par{s0, s1 - 1u};
    }
    const Par inc = wave_par_incl(own);
    if (lane == 63) {
      wt[2 * wv] = inc.a0;
      wt[2 * wv + 1] = inc.a1;
    }
    Par ex = dpp_par<0x138, 0xf, true>(inc);  // wave_shr:1, lane 0 reads (0, 0)
    __syncthreads();
    Par pre{0u, 0u}, tot{0u, 0u};
#pragma unroll
    for (uint32_t i = 0; i < NW; ++i) {
      const Par wtot{wt[2 * i], wt[2 * i + 1]};
      if (i < wv) pre = par_then(pre, wtot);
      tot = par_then(tot, wtot);
    }
    uint64_t cand = ~0ull;
    if (!wave_done) {
      ex = par_then(pre, ex);
      uint32_t cur = C + ((C & 1u) ? ex.a1 : ex.a0);
#pragma unroll
      for (uint32_t q = 0; q < Q; ++q) {
        if (q < nq) {
          const uint32_t t = (tie >> q) & 1u;
          const uint32_t nx = cur + r[q] + (t & ((cur ^ r[q]) & 1u));
          if (cand == ~0ull && Q * tid + q >= s) {
            if (nx >= TOP) {
              // the addition that leaves the binade, as one f32 addition
              const float before = __builtin_ldexpf((float)cur, eb - 23);
              cand = ((uint64_t)(Q * tid + q) << 32) | __float_as_uint(before + e[q]);
            } else if (STOPS) {
              const float cv = __builtin_ldexpf((float)nx, eb - 23);  // exact
              if (cv >= thr) cand = ((uint64_t)(Q * tid + q) << 32) | __float_as_uint(cv);
            }
          }
          cur = nx;
        }
      }
    }
    cand = wave_min_key(cand);
    if (lane == 0 && cand != ~0ull) __atomic_fetch_min(slot, cand, __ATOMIC_RELAXED);
    __syncthreads();
    const uint64_t res = *slot;
    if (res == ~0ull) {
      ++it;
      return __builtin_ldexpf((float)(C + ((C & 1u) ? tot.a1 : tot.a0)), eb - 23);
    }
    c = __uint_as_float((uint32_t)res);
    s = (uint32_t)(res >> 32) + 1u;
    if (STOPS && c >= thr) {
      stop_at = s - 1u;
      ++it;
      return c;
    }
    if (s >= NT * Q) {
      ++it;
      return c;
    }
  }
}
__device__ __forceinline__ float block_seq_sum(const float (&e)[16], uint32_t nq, float c,
                                               uint32_t& it, LDS uint32_t* sc) {
  uint32_t st;
  return block_seq_scan<false>(e, nq, c, it, sc, 0.0f, st);
}

// seq_scan's running sums of list[0..n) (mode 0: the total; 1 and 2: the
// first j whose running sum reaches thr) by the whole workgroup, for long
// lists (the slow path's nuclei): windows of NT*16 entries, thread t holding
// entries 16t .. 16t+15 of a window, each window through block_seq_scan.
// Returns (the stop index, n if none; the running sum there, the total if
// none).  sc: 6 + NW*2 words.  A call of its own, its registers apart from
// the kernel's.
__device__ __attribute__((noinline)) u2v block_list_scan(List list, uint32_t n, int mode,
                                                        float thr, LDS uint32_t* sc) {
  constexpr uint32_t Q = 16;
  const uint32_t tid = threadIdx.x;
  const bool stops = mode != 0;
  if (n > 0 && stops && thr <= 0.0f) return u2v{0u, __float_as_uint(0.0f + list.get(0))};
  if (tid < 3) ((LDS uint64_t*)sc)[tid] = ~0ull;  // the event slots start cleared
  __syncthreads();
  uint32_t it = 0, stop = n;
  float c = 0.0f;
  for (uint32_t w0 = 0; w0 < n; w0 += NT * Q) {
    float e[Q];
#pragma unroll
    for (uint32_t q = 0; q < Q; ++q) {
      const uint32_t i = w0 + Q * tid + q;
      e[q] = i < n ? list.get(i) : 0.0f;
    }
    uint32_t st;
    c = stops ? block_seq_scan<true>(e, Q, c, it, sc, thr, st)
              : block_seq_scan<false>(e, Q, c, it, sc, 0.0f, st);
    if (st != EMPTY) {
      stop = w0 + st;
      break;
    }
  }
  __syncthreads();  // the caller may reuse sc
  return u2v{stop, __float_as_uint(c)};
}

// ---------------------------------------------------------------------------
// Sequential f32 sums in binades
// ---------------------------------------------------------------------------
// While a running sum c >= 0 stays in the binade [2^eb, 2^(eb+1)) (below
// 2^-125 the quantum is 2^-149 throughout) it is an integer C of quanta
// q = 2^(eb-23), C < 2^24, and adding a term p adds round(p / q) quanta, a
// tie going to the even sum: the increment of a run of terms depends on C
// only through its parity, so a run is a pair of increments (from an even,
// from an odd C), and runs compose in order.  An increment that would take C
// to 2^24 or beyond leaves the binade; it saturates at XS_SAT, and the run is
// then taken apart.
constexpr uint32_t XS_SAT = 1u << 24;
__device__ __forceinline__ Par sat_then(Par f, Par g) {
  const uint32_t a0 = f.a0 + ((f.a0 & 1u) ? g.a1 : g.a0);
  const uint32_t a1 = f.a1 + ((f.a1 & 1u) ? g.a0 : g.a1);
  return Par{umin(a0, XS_SAT), umin(a1, XS_SAT)};
}
__device__ __forceinline__ Par wave_par_incl_sat(Par x) {
  x = sat_then(dpp_par<0x111, 0xf, true>(x), x);
  x = sat_then(dpp_par<0x112, 0xf, true>(x), x);
  x = sat_then(dpp_par<0x114, 0xf, true>(x), x);
  x = sat_then(dpp_par<0x118, 0xf, true>(x), x);
  x = sat_then(dpp_par<0x142, 0xa, false>(x), x);
  x = sat_then(dpp_par<0x143, 0xc, false>(x), x);
  return x;
}
// binade exponent of a positive normal or subnormal float (subnormals: -126)
__device__ __forceinline__ int binade_of(float c) {
  return (int)umax((__float_as_uint(c) >> 23) & 255u, 1u) - 127;
}
// floor(log2 x) of a positive normal double
__device__ __forceinline__ int binade_d(double x) {
  return (int)(((uint64_t)__double_as_longlong(x) >> 52) & 0x7ffu) - 1023;
}
// The pair of a lane's Q consecutive terms (>= 0) in the binade of exponent eb.
template <int Q>
__device__ __forceinline__ Par lane_pair(const float (&e)[Q], int eb) {
  uint32_t s0 = 0, s1 = 1;
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const float x = __builtin_fminf(__builtin_ldexpf(e[q], 23 - eb), 0x1p25f);
    const float k = __builtin_floorf(x);
    const float fr = x - k;
    const uint32_t ki = (uint32_t)k;
    const uint32_t r = fr > 0.5f ? ki + 1u : ki;
    const uint32_t t = fr == 0.5f ? 1u : 0u;
    s0 += r + (t & ((s0 ^ r) & 1u));
    s1 += r + (t & ((s1 ^ r) & 1u));
  }
  return Par{umin(s0, XS_SAT), umin(s1 - 1u, XS_SAT)};
}

// c + the terms of lanes pos .. nl - 1 of a wave in order, exactly (lane l
// holding terms Q l .. Q l + Q - 1, zeros past the count), by rounds: a lane
// at a time while c is 0 (from 0 the sum leaves its binade at almost every
// term); then the lanes' pairs in c's binade, a wave scan; the lanes before
// the first one where c leaves the binade are added by their pairs, that
// lane's terms one f32 addition each, and the scan resumes after it.  Every
// lane returns the sum.
// c + lane j's Q terms in order, one f32 addition each, added by lane j
// itself (a chain of register additions; read lane by lane into scalar
// registers the same chain is several times slower); j wave-uniform, every
// lane returns the sum.
template <int Q>
__device__ __forceinline__ float lane_chain(float c, const float (&p)[Q], uint32_t j) {
  float x = c;
  if ((threadIdx.x & 63u) == j) {
#pragma unroll
    for (int q = 0; q < Q; ++q) x = x + p[q];
  }
  return rl(x, j);
}
template <int Q>
__device__ __forceinline__ float wave_sum_rounds(float c, const float (&p)[Q], uint32_t nl,
                                                 uint32_t pos) {
  const uint32_t lane = threadIdx.x & 63u;
  while (pos < nl) {
    if (c == 0.0f) {
      c = lane_chain<Q>(c, p, pos);  // zeros past n add nothing
      ++pos;
      continue;
    }
    const int eb = binade_of(c);
    const uint32_t C = (uint32_t)__builtin_ldexpf(c, 23 - eb);
    Par x = Par{0u, 0u};
    if (lane >= pos) x = lane_pair<Q>(p, eb);
    const Par in = wave_par_incl_sat(x);
    const uint32_t inc = (C & 1u) ? in.a1 : in.a0;
    const uint64_t cross = __ballot(lane >= pos && lane < nl && C + inc >= XS_SAT);
    if (cross == 0ull) {
      c = __builtin_ldexpf((float)(C + (uint32_t)__builtin_amdgcn_readlane((int)inc, 63)), eb - 23);
      break;
    }
    const uint32_t l = (uint32_t)__builtin_ctzll(cross);
    const uint32_t Cb = l > pos ? C + (uint32_t)__builtin_amdgcn_readlane((int)inc, (int)l - 1) : C;
    c = lane_chain<Q>(__builtin_ldexpf((float)Cb, eb - 23), p, l);
    pos = l + 1;
  }
  return c;
}

// The runs of a wave's terms (lane l holding terms Q l .. Q l + Q - 1, zeros
// from lane nl on) for a running sum that enters them anywhere in [clo, chi].
// Each lane bounds the running sums over its terms from those bounds and the
// exact prefix of the lanes' sums: the sequential f32 sum of k positive terms
// from c is within k u (1.001) of the exact one (u = 2^-24 per addition; plus
// 2^-150 per addition below 2^-126), and a lane's own f32 sum within Q u of
// its terms'.  A lane whose bounds share one binade forms its pair there;
// consecutive such lanes of one binade form a run, and a segmented wave scan
// gives each lane its run's pair so far.  RunLane.k: the lane's binade + 512
// (0: no run, the lane is summed one addition a term), bit 16 set where a
// run (or such a lane) starts.
struct RunLane {
  uint32_t a0, a1, k;
};
template <int Q>
__device__ __forceinline__ RunLane seg_runs(const float (&p)[Q], uint32_t nl, double clo,
                                            double chi) {
  const uint32_t lane = threadIdx.x & 63u;
  float ls = 0.0f;
#pragma unroll
  for (int q = 0; q < Q; ++q) ls += p[q];
  const double lsd = (double)ls;
  const double pre = wave_prefix_d(lsd) - lsd;
  const double d = (double)(Q * (lane + 2u) + 4u) * 0x1p-24 * 1.02 + 0x1p-45;
  const double ab = (double)(Q * (lane + 1u)) * 0x1p-150;
  const double lo = (clo + pre) * (1.0 - d) - ab, hi = (chi + pre + lsd) * (1.0 + d) + ab;
  const int eb = binade_d(lo);
  const bool ok = lane < nl && lo >= 0x1p-126 && hi < 0x1p120 && binade_d(hi) == eb;
  const uint32_t key = ok ? (uint32_t)(eb + 512) : 0u;
  const uint32_t prev =
      (uint32_t)__builtin_amdgcn_ds_bpermute((int)(((lane + 63u) & 63u) * 4u), (int)key);
  const bool head = !ok || lane == 0 || prev != key;
  const uint64_t heads = __ballot(head);
  // each lane's run start, then the pairs scanned within runs
  const uint32_t rs = 63u - (uint32_t)__builtin_clzll(heads & ((2ull << lane) - 1ull));
  Par x = lane_pair<Q>(p, ok ? eb : 0);
  Par y = sat_then(dpp_par<0x111, 0xf, true>(x), x);
  x = rs + 1u <= lane ? y : x;
  y = sat_then(dpp_par<0x112, 0xf, true>(x), x);
  x = rs + 2u <= lane ? y : x;
  y = sat_then(dpp_par<0x114, 0xf, true>(x), x);
  x = rs + 4u <= lane ? y : x;
  y = sat_then(dpp_par<0x118, 0xf, true>(x), x);
  x = rs + 8u <= lane ? y : x;
  y = sat_then(dpp_par<0x142, 0xa, false>(x), x);
  x = rs + 1u <= (lane & ~15u) ? y : x;
  y = sat_then(dpp_par<0x143, 0xc, false>(x), x);
  x = rs <= 31u ? y : x;
  return RunLane{x.a0, x.a1, key | (head ? 0x10000u : 0u)};
}
// c + the terms of lanes 0 .. nl - 1 in order, exactly, c inside the bounds
// r was formed for: a run at once (its sum provably stays in its binade),
// every other lane (a binade crossing, or c = 0) one f32 addition a term.
// Where the sum is not where the bounds say (it cannot be; the check keeps
// the result exact whatever), the rest goes by rounds (wave_sum_rounds).
// Every lane returns the sum.
template <int Q>
__device__ __forceinline__ float runs_walk(float c, const float (&p)[Q], uint32_t nl, RunLane r) {
  const uint64_t heads = __ballot((r.k >> 16) & 1u);
  const uint64_t bad = __ballot((r.k & 0xffffu) == 0u);
  uint32_t pos = 0;
  while (pos < nl) {
    if ((bad >> pos) & 1ull) {
      c = lane_chain<Q>(c, p, pos);
      ++pos;
      continue;
    }
    const uint64_t after = heads & ~((2ull << pos) - 1ull);
    const uint32_t end = after ? (uint32_t)__builtin_ctzll(after) : 64u;
    const uint32_t last = (end < nl ? end : nl) - 1u;
    const int ebr = (int)((uint32_t)__builtin_amdgcn_readlane((int)r.k, (int)pos) & 0xffffu) - 512;
    if (!(c >= 0x1p-126f) || binade_of(c) != ebr) break;
    const uint32_t C = (uint32_t)__builtin_ldexpf(c, 23 - ebr);
    const uint32_t inc = (C & 1u) ? (uint32_t)__builtin_amdgcn_readlane((int)r.a1, (int)last)
                                  : (uint32_t)__builtin_amdgcn_readlane((int)r.a0, (int)last);
    if (C + inc >= XS_SAT) break;
    c = __builtin_ldexpf((float)(C + inc), ebr - 23);
    pos = last + 1u;
  }
  return pos < nl ? wave_sum_rounds<Q>(c, p, nl, pos) : c;
}
// c + the first n of a wave's terms in order, exactly, by their runs from c.
template <int Q>
__device__ __forceinline__ float wave_sum_q(float c, const float (&p)[Q], uint32_t n) {
  const uint32_t nl = (n + Q - 1) / Q;  // lanes holding terms
  if (nl == 0) return c;
  return runs_walk<Q>(c, p, nl, seg_runs<Q>(p, nl, (double)c, (double)c));
}

// A wave-uniform 64-bit value, or LDS pointer, in scalar registers.
__device__ __forceinline__ uint64_t sgpr_u64(uint64_t x) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)x);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(x >> 32));
  return ((uint64_t)hi << 32) | lo;
}
template <class T>
__device__ __forceinline__ LDS T* sgpr_lds(LDS T* p) {
  const uint32_t a = (uint32_t)(uintptr_t)p;
  return (LDS T*)(uintptr_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)a);
}

// S = the sequential f32 sum in index order of e_i = exp_ref(fl(l_i - m))
// (0 for l_i = -inf), l_i = fl(v_i / T) the processed logit (penalties from
// the history tables h if have_hist, the allow-mask, NaN read as -inf)
// divided by T (sampler.rs:53, :57-66).  The whole workgroup, in windows of
// NT*16 consecutive elements, thread t holding elements 16t .. 16t+15 of a
// window (wave w: its 1024-element segment w); the next window's logits are
// requested before the current one is summed.
//
// Most elements cannot change the sum: zeros (-inf logits), and, once the sum
// is positive, every e below half its quantum at the window's start (the sum
// only grows, so such an e adds 0 wherever it falls).  A cheap bound on l
// finds them (the product with 1/T is within a few ulps of l, far inside the
// margin).  A wave whose segment keeps at most 256 (its live terms) packs
// them in order into LDS, so that the exact division and exp run on those
// alone, and goes on with them four a lane; any other keeps its sixteen a
// lane (dead ones 0).
//
// Then each wave predicts the binades its segment's running sum occupies,
// from the window's exact starting sum and the segments' sums (within the
// drift n u of an f32 sum of n terms), and sums its terms in pairs in each
// (at most three); wave 0 walks the sixteen segments with the exact running
// sum: a run of segments whose pair covers the sum's binade and keeps it
// there is added at once; a segment where the sum leaves its binade, or that
// no pair covers, is summed by the wave that holds it (wave_sum_q), at wave
// 0's request through LDS.  The sum is exact whatever the predictions; they
// only decide how much is summed lane by lane.  sc: XS_SC words of scratch.
// A function of its own (not inlined, scalars only across the call): its
// registers are then allocated apart from the stream loop's, which an
// inlined copy crowds into spilling.
constexpr uint32_t XS_NB = 3;                    // binades summarised per segment
constexpr uint32_t XS_CW = 256;                  // live terms a wave packs
constexpr uint32_t XS_SC = 136 + NW * XS_CW;     // scratch words
template <int DT>
__device__ __attribute__((noinline)) float exact_normaliser(
    const void* row, const uint32_t* mask_row, uint32_t V, float T, float m,
    LDS uint32_t* bitmap, LDS uint16_t* pre, LDS float* pen, bool have_hist, LDS uint32_t* sc) {
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  // the arguments arrive in vector registers; the row's pointers, the LDS
  // tables and the scalars are moved to scalar ones, which the window loop
  // then does not spill (a reload from scratch waits for every load in
  // flight, the next window's logits among them)
  const uint32_t wv = (uint32_t)__builtin_amdgcn_readfirstlane((int)(tid >> 6));
  sc = sgpr_lds(sc);
  bitmap = sgpr_lds(bitmap);
  pre = sgpr_lds(pre);
  pen = sgpr_lds(pen);
  row = (const void*)sgpr_u64((uint64_t)row);
  mask_row = (const uint32_t*)sgpr_u64((uint64_t)mask_row);
  T = __uint_as_float((uint32_t)__builtin_amdgcn_readfirstlane((int)__float_as_uint(T)));
  m = __uint_as_float((uint32_t)__builtin_amdgcn_readfirstlane((int)__float_as_uint(m)));
  V = (uint32_t)__builtin_amdgcn_readfirstlane((int)V);
  const GLB uint32_t* mrow = mask_row ? G(mask_row) : nullptr;
  Hist h;
  h.bitmap = bitmap;
  h.pre = pre;
  h.pen = pen;
  h.tokr = nullptr;
  h.lo = 0;
  constexpr uint32_t Q = 16, W = NT * Q, CW = XS_CW;
  enum : uint32_t { REQ = 0, CV = 1, ACK = 2, CEND = 3 };
  constexpr uint32_t FINISHED = 0xfffffffeu;
  LDS uint32_t* segp = sc;                         // [NW][7]: binades, three pairs
  LDS float* wsum = (LDS float*)(sc + 112);        // [NW]: the segments' sums
  LDS uint32_t* ctl = sc + 128;                    // the walk's requests
  LDS float* comp = (LDS float*)(sc + 136) + CW * wv;  // this wave's packed terms
  const float rT = 1.0f / T;
  auto exact_e = [&](float x) __attribute__((always_inline)) {
    const float l = (T != 1.0f) ? x / T : x;
    return (l == NEG_INF) ? 0.0f : exp_ref<true>(l - m);
  };
  float c = 0.0f;
  float xn[Q];
  load16<DT>(row, Q * tid, V, xn);
  // the mask word of the next window, requested with its logits
  uint32_t mwn = (mrow && Q * tid < V) ? mrow[(Q * tid) >> 5] : 0xffffffffu;
  for (uint32_t w0 = 0; w0 < V; w0 += W) {
    const uint32_t e0 = w0 + Q * tid;
    float x[Q];
#pragma unroll
    for (uint32_t q = 0; q < Q; ++q) x[q] = xn[q];
    // the sixteen lie in one 32-bit word of the mask and of the bitmap
    const uint32_t mw = mwn >> (e0 & 16u);
    const uint32_t hw = (have_hist && e0 < V) ? h.bitmap[(e0 - h.lo) >> 5] >> (e0 & 16u) : 0u;
    // entries below lim (on l - m) add nothing to a sum of binade eb or above
    float lim = NEG_INF;
    if (c > 0.0f) lim = (float)(binade_of(c) - 24) * 0.693147f - (0.01f + 1e-6f * fabsf(m));
    uint32_t live = 0;
#pragma unroll
    for (uint32_t q = 0; q < Q; ++q) {
      float v = x[q];
      if ((hw >> q) & 1u) v = h.pen[h.rank(e0 + q)];  // a kept rank (< U_MAX)
      if (!((mw >> q) & 1u) || !(v > NEG_INF)) v = NEG_INF;
      x[q] = v;
      if (v > NEG_INF && v * rT - m >= lim) live |= 1u << q;
    }
    // the next window's logits and mask word, while this one is summed
    if (w0 + W < V) {
      load16<DT>(row, e0 + W, V, xn);
      if (mrow && e0 + W < V) mwn = mrow[(e0 + W) >> 5];
    }
    // ---- the exact terms: packed (four a lane, in order) or sixteen a lane
    const uint32_t n = (uint32_t)__popc(live);
    const uint32_t incl = wave_incl_scan(n);
    const uint32_t nw = bcast63u(incl);
    const bool packed = nw <= CW;  // wave-uniform
    float e[Q];
    float pk[4];
    if (packed) {
      uint32_t at = incl - n;
#pragma unroll
      for (uint32_t q = 0; q < Q; ++q)
        if ((live >> q) & 1u) comp[at++] = x[q];
      WaveSync::sync();
#pragma unroll
      for (uint32_t k = 0; k < CW / WAVE; ++k) {
        const uint32_t i = lane + WAVE * k;
        if (WAVE * k < nw && i < nw) comp[i] = exact_e(comp[i]);
      }
      WaveSync::sync();
      const f4v v4 = ((LDS const f4v*)comp)[lane];
      pk[0] = 4 * lane + 0 < nw ? v4.x : 0.0f;
      pk[1] = 4 * lane + 1 < nw ? v4.y : 0.0f;
      pk[2] = 4 * lane + 2 < nw ? v4.z : 0.0f;
      pk[3] = 4 * lane + 3 < nw ? v4.w : 0.0f;
    } else {
#pragma unroll
      for (uint32_t q = 0; q < Q; ++q) e[q] = ((live >> q) & 1u) ? exact_e(x[q]) : 0.0f;
    }
    // the terms a segment holds: nw packed, else the elements in V
    const uint32_t sbase = w0 + TILE * wv;
    const uint32_t nseg = packed ? nw : (sbase < V ? umin(TILE, V - sbase) : 0u);
    // ---- the segment's sum, then the binades its running sum occupies
    float ls = 0.0f;
    if (packed) {
      ls = (pk[0] + pk[1]) + (pk[2] + pk[3]);
    } else {
#pragma unroll
      for (uint32_t q = 0; q < Q; ++q) ls += e[q];
    }
    ls = wave_tree_sum(ls);
    if (lane == 0) wsum[wv] = ls;
    if (tid == 0) {
      ctl[REQ] = EMPTY;
      ctl[ACK] = EMPTY;
    }
    __syncthreads();
    double before = (double)c;
    for (uint32_t i = 0; i < wv; ++i) before += (double)wsum[i];
    // the drift of an f32 sum of n terms (n: the window's elements up to
    // this segment's end) and of the segments' f32 sums
    const double drift = (double)(TILE * (wv + 1)) * 0x1p-24 * 1.01 + 0x1p-19;
    const double plo = before * (1.0 - drift), phi = (before + (double)wsum[wv]) * (1.0 + drift);
    uint32_t hdr = 0;  // eb_lo + 256 in bits 0..15, binades in 16..23 (0: no pairs)
    Par pr[XS_NB];
#pragma unroll
    for (uint32_t k = 0; k < XS_NB; ++k) pr[k] = Par{0u, 0u};
    if (plo >= 0x1p-126 && phi < 0x1p120) {
      const int elo = binade_d(plo), ehi = binade_d(phi);
      const int nb = ehi - elo + 1;
      if (nb <= (int)XS_NB) {
#pragma unroll
        for (int k = 0; k < (int)XS_NB; ++k) {
          if (k < nb) {
            const Par y = packed ? wave_par_incl_sat(lane_pair<4>(pk, elo + k))
                                 : wave_par_incl_sat(lane_pair<Q>(e, elo + k));
            pr[k] = Par{(uint32_t)__builtin_amdgcn_readlane((int)y.a0, 63),
                        (uint32_t)__builtin_amdgcn_readlane((int)y.a1, 63)};
          }
        }
        hdr = (uint32_t)(elo + 256) | ((uint32_t)nb << 16);
      }
    }
    if (lane == 0) {
      segp[7 * wv] = hdr;
#pragma unroll
      for (uint32_t k = 0; k < XS_NB; ++k) {
        segp[7 * wv + 1 + 2 * k] = pr[k].a0;
        segp[7 * wv + 2 + 2 * k] = pr[k].a1;
      }
    }
    __syncthreads();
    // ---- the walk
    if (wv == 0) {
      float cc = c;
      uint32_t s = 0;
      while (s < (uint32_t)NW) {
        if (__float_as_uint(cc) >= 0x00800000u) {
          // segments s .. s + g - 1 keep the sum in its binade (a prefix of the lanes)
          const int eb = binade_of(cc);
          const uint32_t C = (uint32_t)__builtin_ldexpf(cc, 23 - eb);
          const uint32_t j = s + lane;
          Par px = Par{XS_SAT, XS_SAT};
          if (j < (uint32_t)NW) {
            const uint32_t hj = segp[7 * j];
            const int k = eb - ((int)(hj & 0xffffu) - 256);
            if ((hj >> 16) != 0u && k >= 0 && k < (int)(hj >> 16))
              px = Par{segp[7 * j + 1 + 2 * k], segp[7 * j + 2 + 2 * k]};
          }
          const Par in = wave_par_incl_sat(px);
          const uint32_t inc = (C & 1u) ? in.a1 : in.a0;
          const uint64_t good = __ballot(j < (uint32_t)NW && C + inc < XS_SAT);
          const uint32_t g = ~good == 0ull ? 64u : (uint32_t)__builtin_ctzll(~good);
          if (g > 0) {
            const uint32_t ig = (uint32_t)__builtin_amdgcn_readlane((int)inc, (int)g - 1);
            cc = __builtin_ldexpf((float)(C + ig), eb - 23);
            s += g;
            continue;
          }
        }
        // segment s, lane by lane, by the wave that holds it
        if (s == 0) {
          cc = packed ? wave_sum_rounds<4>(cc, pk, (nseg + 3u) / 4u, 0u)
                      : wave_sum_rounds<Q>(cc, e, (nseg + Q - 1u) / Q, 0u);
        } else {
          if (lane == 0) {
            __hip_atomic_store(&ctl[CV], __float_as_uint(cc), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
            __hip_atomic_store(&ctl[REQ], s, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
          }
          while (__hip_atomic_load(&ctl[ACK], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) != s)
            __builtin_amdgcn_s_sleep(1);
          cc = __uint_as_float(
              __hip_atomic_load(&ctl[CV], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
        }
        ++s;
      }
      if (lane == 0) {
        ctl[CEND] = __float_as_uint(cc);
        __hip_atomic_store(&ctl[REQ], FINISHED, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    } else {
      // until wave 0 asks for this segment or has walked the window
      for (;;) {
        const uint32_t r =
            __hip_atomic_load(&ctl[REQ], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (r == wv) {
          const float cin = __uint_as_float(
              __hip_atomic_load(&ctl[CV], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
          const float cout = packed ? wave_sum_rounds<4>(cin, pk, (nseg + 3u) / 4u, 0u)
                                    : wave_sum_rounds<Q>(cin, e, (nseg + Q - 1u) / Q, 0u);
          if (lane == 0) {
            __hip_atomic_store(&ctl[CV], __float_as_uint(cout), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
            __hip_atomic_store(&ctl[ACK], wv, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
          }
          break;
        }
        if (r == FINISHED) break;
        __builtin_amdgcn_s_sleep(1);
      }
    }
    __syncthreads();
    c = __uint_as_float(ctl[CEND]);
    __syncthreads();  // ctl, segp, wsum and comp are rewritten next window
  }
  return c;
}

// ---------------------------------------------------------------------------
// Slow path (one workgroup, one row)
// ---------------------------------------------------------------------------
// Eight consecutive logits of a row from e0 (zeros past V).
template <int DT>
__device__ __forceinline__ void load8(const void* row, uint32_t e0, uint32_t V, float x[8]) {
  if (e0 + 8 <= V) {
    if ((DT & 3) == LLMK_F32) {
      const GLB f4v* r = (const GLB f4v*)((const GLB float*)row + e0);
      const f4v a = r[0], b = r[1];
      x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
      x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    } else {
      const GLB u2v* r = (const GLB u2v*)((const GLB uint16_t*)row + e0);
      const u2v a = r[0], b = r[1];
      const uint32_t w[4] = {a.x, a.y, b.x, b.y};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        x[2 * q] = cvt16<DT>(w[q] & 0xffffu);
        x[2 * q + 1] = cvt16<DT>(w[q] >> 16);
      }
    }
    if (DT & SOFTCAP) {
#pragma unroll
      for (int q = 0; q < 8; ++q) x[q] = softcap<DT>(x[q]);
    }
  } else {
#pragma unroll
    for (int q = 0; q < 8; ++q) x[q] = e0 + q < V ? load_logit<DT>(row, e0 + q) : 0.0f;
  }
}

// Stable LSD radix sort of src[0..npos) on bits 32..63 of the keys, four
// passes of 8 bits through dst (src holds the sorted keys after the even
// number of passes), by the whole workgroup.  Inlined: as a call of its
// own it measured C5 1.5 us slower (the stream kernel's code moves).
// wcnt: NW*256 words, digit_off: 256, red: 64.
__device__ __forceinline__ void radix_sort_keys(GLB uint64_t* src, GLB uint64_t* dst,
                                                         uint32_t npos, LDS uint32_t* wcnt,
                                                         LDS uint32_t* digit_off,
                                                         LDS uint32_t* red) {
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wv = (uint32_t)__builtin_amdgcn_readfirstlane((int)(tid >> 6));
  src = (GLB uint64_t*)sgpr_u64((uint64_t)src);
  dst = (GLB uint64_t*)sgpr_u64((uint64_t)dst);
  npos = (uint32_t)__builtin_amdgcn_readfirstlane((int)npos);
  for (uint32_t j = tid; j < NW * 256; j += NT) wcnt[j] = 0;
  for (int pass = 0; pass < 4; ++pass) {
    const int sh_bits = 32 + 8 * pass;
    if (tid < 256) digit_off[tid] = 0;
    __syncthreads();
    // the digit histogram, RE keys per thread loaded at once: a wave whose
    // keys share one digit (the top digits of p keys are few and equal, and
    // per-element atomics on one address serialise) adds its count once
    constexpr int RE = 8;
    for (uint32_t b0 = 0; b0 < npos; b0 += RE * NT) {
      uint32_t dg[RE];
#pragma unroll
      for (int q = 0; q < RE; ++q) {
        const uint32_t i = b0 + q * NT + tid;
        dg[q] = i < npos ? (uint32_t)(src[i] >> sh_bits) & 255u : 256u;
      }
#pragma unroll
      for (int q = 0; q < RE; ++q) {
        if (b0 + q * NT >= npos) break;
        // the valid lanes are a prefix of the wave: lane 0 holds one if any
        // does; a wave of one digit (the high digits of p keys) adds its
        // count once, any other adds per lane (spread digits rarely collide)
        const bool valid = dg[q] < 256u;
        const uint32_t d0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)dg[q]);
        const uint64_t vm = __ballot(valid);
        if (__ballot(valid && dg[q] != d0) == 0) {
          if (lane == 0 && vm)
            __atomic_fetch_add(&digit_off[d0 & 255u], (uint32_t)__popcll(vm), __ATOMIC_RELAXED);
        } else if (valid) {
          __atomic_fetch_add(&digit_off[dg[q]], 1u, __ATOMIC_RELAXED);
        }
      }
    }
    __syncthreads();
    // exclusive prefix of the 256 digit counts: waves 0..3, one digit a lane
    {
      const uint32_t c = tid < 256 ? digit_off[tid] : 0u;
      const uint32_t incl = wave_incl_scan(c);
      if (tid < 256 && lane == 63) red[wv] = incl;
      __syncthreads();
      if (tid < 256) {
        uint32_t base = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) base += q < wv ? red[q] : 0u;
        digit_off[tid] = base + incl - c;
      }
    }
    __syncthreads();
    // stable scatter, RE * NT keys per step: wave w ranks its own run of
    // RE * 64 consecutive keys slot after slot (equal digits found by
    // ballots, counted on in the wave's row of wcnt), then one prefix per
    // digit across the waves (written over the counts) places every key;
    // each wave reads only its own row when it scatters and clears it
    // after, so two barriers per step
    for (uint32_t b0 = 0; b0 < npos; b0 += RE * NT) {
      const uint32_t wb = b0 + (uint32_t)wv * (RE * WAVE);
      uint64_t ky[RE];
      uint32_t pw[RE];
#pragma unroll
      for (int q = 0; q < RE; ++q) {
        const uint32_t i = wb + q * WAVE + lane;
        ky[q] = i < npos ? src[i] : 0ull;
      }
#pragma unroll
      for (int q = 0; q < RE; ++q) {
        const bool valid = wb + q * WAVE + lane < npos;
        const uint32_t d = (uint32_t)(ky[q] >> sh_bits) & 255u;
        uint64_t peers = __ballot(valid);
        pw[q] = 0;
        if (peers == 0) continue;  // wave-uniform: this slot is past the keys
        // the lanes holding this lane's digit: all valid lanes when the wave
        // holds one digit, else matched bit by bit
        const uint32_t d0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)d);
        if (__ballot(valid && d != d0) != 0) {
#pragma unroll
          for (int bit = 0; bit < 8; ++bit) {
            const uint64_t bb = __ballot(((d >> bit) & 1u) != 0);
            peers &= ((d >> bit) & 1u) ? bb : ~bb;
          }
        }
        const uint32_t rank = lanes_below(peers);
        const uint32_t base = valid ? wcnt[wv * 256 + d] : 0u;
        pw[q] = base + rank;
        WaveSync::sync();  // every lane has read the count before it moves on
        if (valid && rank == 0) wcnt[wv * 256 + d] = base + (uint32_t)__popcll(peers);
        WaveSync::sync();  // the next slot reads the new counts
      }
      __syncthreads();
      if (tid < 256) {
        // the sixteen counts read at once, then the prefix
        uint32_t c[NW];
#pragma unroll
        for (int w2 = 0; w2 < NW; ++w2) c[w2] = wcnt[w2 * 256 + tid];
        uint32_t acc = digit_off[tid];
#pragma unroll
        for (int w2 = 0; w2 < NW; ++w2) {
          wcnt[w2 * 256 + tid] = acc;
          acc += c[w2];
        }
        digit_off[tid] = acc;
      }
      __syncthreads();
#pragma unroll
      for (int q = 0; q < RE; ++q) {
        if (wb + q * WAVE + lane < npos) {
          const uint32_t d = (uint32_t)(ky[q] >> sh_bits) & 255u;
          dst[wcnt[wv * 256 + d] + pw[q]] = ky[q];
        }
      }
      WaveSync::sync();  // this wave's reads of its row are done
#pragma unroll
      for (int w2 = 0; w2 < 4; ++w2) wcnt[wv * 256 + 64 * w2 + lane] = 0;
    }
    wait_stores();
    __syncthreads();
    if (tid == 0) __threadfence();
    __syncthreads();
    GLB uint64_t* tmp = src;
    src = dst;
    dst = tmp;
  }
}

// ---------------------------------------------------------------------------
// Slow path (one workgroup, one row).  Rows the candidate path cannot prove:
//   A  every processed logit l falls in a bin of d = (l - L) log2(e)/T (1/16
//      per bin, the last bin open-ended), counted in LDS;
//   B  the bins that the semantics can reach are chosen from those counts:
//      the first bins (largest l) whose lower bound on sum 2^d reaches
//      (top_p, or the uniform when top-p is off) * S + 0.002 S, and for a
//      top-k row the first bins holding K elements -- a guess, checked
//      below;
//   C  the exact p of every element of the chosen bins, kept in index order
//      (p > 0 as (p, idx) keys, p == 0 as indices when nothing is left out);
//      the largest logit left out bounds the p of everything left out
//      (p_lim);
//   D  a stable LSD radix sort of the keys, then min-p / top-k / top-p / the
//      draw over the sorted list, whose exact prefix is the entries with
//      p > p_lim.  If the semantics need an entry past it, C and D are done
//      again with every bin chosen.
// ---------------------------------------------------------------------------
// approx: S = 1 stands in for the reference's S (a row that top-k
// renormalises); its result stands only if the band check proves it, else S
// is computed (exact_normaliser) and the row sampled again.  need_exact: S is
// computed first (the candidate path's band check already failed, or the row
// has no top-k).
//
// MAT: the row's history holds more distinct tokens than the LDS tables
// (U_MAX ranks), so the row is first materialised: its processed logits
// (softcap, penalties by each token's count, the allow-mask, NaN as -inf)
// into the slot's scratch, the counts gathered there with global atomics;
// every pass then reads them from there (sampler.rs:132-146 has no limit on
// the history), and the row's maximum is taken again from them.  Without
// MAT, a row whose tables overflow returns true at once (nothing written):
// the caller runs it again with MAT.
template <int DT, bool MAT>
__device__ __forceinline__ bool slow_row(const Args& a, const Ws& w, uint32_t b, const RowP& P,
                                         float S, float m, float L, LDS uint32_t* smem,
                                         bool approx, bool need_exact) {
  const uint32_t tid = threadIdx.x;
  const int lane = (int)(tid & 63), wv = (int)(tid >> 6);
  const uint32_t V = a.V;
  __syncthreads();
  LDS uint32_t* sh = smem;                   // 64
  LDS uint32_t* red = sh + 64;               // 64
  LDS uint32_t* digit_off = red + 64;        // 256
  LDS uint32_t* wcnt = digit_off + 256;      // NW*256
  LDS uint32_t* bins = wcnt + NW * 256;      // SLOW_BINS
  LDS uint32_t* hb = bins + SLOW_BINS;
  const uint32_t nwords = (V + 31) / 32;
  Hist h;
  hist_carve(h, hb, nwords);
  h.lo = 0;
  // Acquire scratch slot b % slow_slots (a row has its own up to 512 rows).
  // A holder waits on nothing, so the wait ends; the spin is bounded all the
  // same.
  const uint32_t slot = b % w.slow_slots;
  if (tid == 0) {
    uint32_t got = 0;
    for (uint32_t n = 0; n < (1u << 26); ++n) {
      if (atomicCAS(&w.slow_lock[slot], 0u, 1u) == 0u) {
        got = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(8);
    }
    if (got) __threadfence();
    sh[63] = got;
  }
  __syncthreads();
  if (!sh[63]) {
    if (tid == 0) {
      a.out_tok[b] = LLMK_INVALID_TOKEN;
      if (a.out_cnt) a.out_cnt[b] = 0;
      atomicOr(w.status, LLMK_STATUS_SLOT_TIMEOUT);
    }
    return false;
  }
  const void* row = (const char*)a.logits +
                    (uint64_t)b * a.stride * ((DT & 3) == LLMK_F32 ? 4u : 2u);
  if (tid == 0) sh[10] = 0;
  build_history<DT>(a, P, b, row, 0, V, nwords, h, red, &sh[10]);
  const uint32_t* mask_row = a.mask ? a.mask + (uint64_t)b * a.mask_words : nullptr;
  GLB uint64_t* kA = G(w.slow_keys) + (uint64_t)slot * 3 * (uint64_t)w.max_vocab;
  GLB uint64_t* kB = kA + w.max_vocab;
  GLB uint32_t* zl = (GLB uint32_t*)(kB + w.max_vocab);  // zero-probability indices
  GLB float* proc = (GLB float*)(zl + w.max_vocab);      // materialised logits (past zl)
  GLB float* plist = G(w.slow_p) + (uint64_t)slot * w.max_vocab;
  GLB uint32_t* ilist = G(w.slow_idx) + (uint64_t)slot * w.max_vocab;
  const GLB uint32_t* mrow = a.mask ? G(a.mask) + (uint64_t)b * a.mask_words : nullptr;
  if (!MAT && (sh[10] & FLAG_HIST_OVERFLOW) != 0) {  // uniform (after the tables' barrier)
    __syncthreads();
    if (tid == 0) {
      __threadfence();
      atomicExch(&w.slow_lock[slot], 0u);
    }
    return true;
  }
  if constexpr (MAT) {
    if (tid == 0) atomicOr(w.status, LLMK_STATUS_HISTORY_OVERFLOW);
    // the counts of the row's history tokens, then the processed logits
    GLB uint32_t* cnt = (GLB uint32_t*)proc;
    for (uint32_t i = tid; i < V; i += NT) cnt[i] = 0;
    __syncthreads();
    const uint32_t h0 = G(a.hoff)[b];
    const uint32_t h1 = a.hlen ? h0 + G(a.hlen)[b] : G(a.hoff)[b + 1];
    for (uint32_t i = h0 + tid; i < h1; i += NT) {
      const uint32_t t = G(a.htok)[i];
      if (t < V)
        __hip_atomic_fetch_add(&cnt[t], hist_weight(a, i), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    __threadfence_block();
    __syncthreads();
    const bool need_cnt = P.fp != 0.0f;
    for (uint32_t e0 = 8 * tid; e0 < V; e0 += 8 * NT) {
      float v[8];
      load8<DT>(row, e0, V, v);
      const uint32_t mw = (mrow && e0 < V) ? mrow[e0 >> 5] : 0xffffffffu;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const uint32_t e = e0 + q;
        if (e >= V) break;
        float x = v[q];
        const uint32_t k = cnt[e];
        if (k) x = penalize(x, P, need_cnt ? k : 1u);
        if (!((mw >> (e & 31)) & 1u) || !(x > NEG_INF)) x = NEG_INF;
        proc[e] = x;
      }
    }
    __threadfence_block();
    __syncthreads();
    // the row's maximum (and first index of it) over the processed logits:
    // the stream phase's, taken with the history cut short, may differ
    float mx = NEG_INF;
    uint32_t mi = EMPTY;
    for (uint32_t e = tid; e < V; e += NT) {
      const float x = proc[e];
      if (x > mx) {
        mx = x;
        mi = e;
      }
    }
    mx = block_max(mx, (LDS float*)red);
    if (!(mi != EMPTY && proc[mi] == mx)) mi = EMPTY;
    mi = block_min_u32(mi, red);
    L = mx;
    m = (P.T != 1.0f) ? L / P.T : L;
    if (L == NEG_INF) S = 0.0f;
    if (P.mode == MODE_GREEDY) {
      // sampler.rs:40-50: the first index holding the maximum
      if (tid == 0) {
        const uint32_t bi = mi == EMPTY ? 0u : mi;
        a.out_tok[b] = bi;
        if (a.out_cnt) a.out_cnt[b] = 1;
        if (a.out_cap) {
          if (a.out_ids) a.out_ids[(uint64_t)b * a.out_cap] = bi;
          if (a.out_probs) a.out_probs[(uint64_t)b * a.out_cap] = 1.0f;
        }
        __threadfence();
        atomicExch(&w.slow_lock[slot], 0u);
      }
      return false;
    }
    if (L == NEG_INF) {
      need_exact = false;
      approx = false;
    }
  }
  if (need_exact) {
    // sh, red, digit_off and wcnt are scratch of the normaliser here
    if constexpr (MAT)
      S = exact_normaliser<LLMK_F32>((const float*)proc, nullptr, V, P.T, m, h.bitmap, h.pre,
                                     h.pen, false, smem);
    else
      S = exact_normaliser<DT>(row, mask_row, V, P.T, m, h.bitmap, h.pre, h.pen, true, smem);
    approx = false;
  }
  const float u = G(a.u)[b];
  const float c2 = LOG2E_F / P.T;
  const float nbL = -(L * c2);
  // processed logits (penalties, mask, NaN as -inf) of e0 .. e0+7 and their bins
  auto processed = [&](uint32_t e0, float v[8]) __attribute__((always_inline)) {
    if constexpr (MAT) {
#pragma unroll
      for (int q = 0; q < 8; ++q) v[q] = e0 + q < V ? proc[e0 + q] : NEG_INF;
      return;
    }
    load8<DT>(row, e0, V, v);
    const uint32_t mw = (mrow && e0 < V) ? mrow[e0 >> 5] : 0xffffffffu;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const uint32_t e = e0 + q;
      float x = v[q];
      if (e < V && ((h.bitmap[e >> 5] >> (e & 31)) & 1u)) {
        const uint32_t r = h.rank(e);
        if (r < U_MAX) x = h.pen[r];
      }
      if (!((mw >> (e & 31)) & 1u)) x = NEG_INF;
      if (!(x > NEG_INF) || e >= V) x = NEG_INF;
      v[q] = x;
    }
  };
  auto bin_of = [&](float x) __attribute__((always_inline)) {
    const float t = -__builtin_fmaf(x, c2, nbL) * 16.0f;
    return (uint32_t)__builtin_fminf(__builtin_fmaxf(t, 0.0f), (float)(SLOW_BINS - 1));
  };
  // ---- A: bin counts
  for (uint32_t j = tid; j < SLOW_BINS; j += NT) bins[j] = 0;
  __syncthreads();
  for (uint32_t b0 = 0; b0 < V; b0 += 8 * NT) {
    float v[8];
    processed(b0 + 8 * tid, v);
#pragma unroll
    for (int q = 0; q < 8; ++q)
      if (v[q] > NEG_INF) __atomic_fetch_add(&bins[bin_of(v[q])], 1u, __ATOMIC_RELAXED);
  }
  __syncthreads();
  // ---- B: the last chosen bin (wave 0; lane l sums bins 32l .. 32l+31)
  if (wv == 0) {
    constexpr uint32_t PER = SLOW_BINS / WAVE;
    const bool topk = P.K > 0 && (uint32_t)P.K < V;
    // the mass rule reads p = e / S, which needs the row's S: rows that top-k
    // renormalises (S = 1) choose by count alone
    const float tm = (P.top_p < 1.0f ? P.top_p : u) + 0.002f;
    const bool use_mass = !topk && tm < 1.0f && S > 0.0f;
    uint32_t cnt = 0;
    float mass = 0.0f;
    for (uint32_t k = 0; k < PER; ++k) {
      const uint32_t bi = PER * (uint32_t)lane + k;
      const uint32_t c = bins[bi];
      cnt += c;
      if (bi + 1 < SLOW_BINS) mass += (float)c * __builtin_exp2f(-(float)(bi + 1) * 0.0625f);
    }
    const uint32_t cincl = wave_incl_scan(cnt);
    float mincl = mass;  // inclusive scan of the lane masses (order fixed)
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const float o = __shfl_up(mincl, d);
      if (lane >= d) mincl += o;
    }
    const float mneed = tm * S;
    uint32_t last = SLOW_BINS - 1;
    const uint64_t hm = use_mass ? __ballot(mincl >= mneed) : 0ull;
    const uint64_t hk = topk ? __ballot(cincl >= (uint32_t)P.K) : 0ull;
    auto bin_in = [&](uint32_t l, bool by_mass) {
      // the first bin of lane l where the running total meets the target
      const uint32_t c0 = (uint32_t)__shfl((int)(cincl - cnt), (int)l);
      const float m0 = __shfl(mincl - mass, (int)l);
      uint32_t cc = c0;
      float mm = m0;
      uint32_t r = PER * l + PER - 1;
      for (uint32_t k = 0; k < PER; ++k) {
        const uint32_t bi = PER * l + k;
        const uint32_t c = bins[bi];
        cc += c;
        if (bi + 1 < SLOW_BINS) mm += (float)c * __builtin_exp2f(-(float)(bi + 1) * 0.0625f);
        if (by_mass ? mm >= mneed : cc >= (uint32_t)P.K) {
          r = bi;
          break;
        }
      }
      return r;
    };
    if (hm) last = umin(last, bin_in((uint32_t)__ffsll((unsigned long long)hm) - 1, true));
    if (hk) last = umin(last, bin_in((uint32_t)__ffsll((unsigned long long)hk) - 1, false));
    // min-p: the chosen bins reach below p_max * min_p (d = log2(min_p)),
    // so that its cut is seen or lies past every chosen entry; the later
    // steps read only what it keeps, so the count and mass rules do not
    // apply to such a row
    if (P.min_p > 0.0f) {
      const float bm = __builtin_ceilf(-16.0f * __builtin_log2f(P.min_p)) + 2.0f;
      last = (uint32_t)__builtin_fminf(__builtin_fmaxf(bm, 0.0f), (float)(SLOW_BINS - 1));
    }
    if (lane == 0) sh[11] = last;
  }
  __syncthreads();
  uint32_t last = sh[11];
  uint32_t tok = 0, len = 0;
  List Lst{flat(plist), flat(ilist), Chain{0.f, 0.f, 0.f, 0}, nullptr};
  // at most: the chosen bins, every bin, then both again with the
  // reference's S when the band check fails
  for (int attempt = 0; attempt < 4; ++attempt) {
    const bool filt = last < SLOW_BINS - 1;
    // ---- C: exact p of the chosen elements, in index order
    uint32_t npos = 0, nzero = 0, lkey = 0;
    for (uint32_t b0 = 0; b0 < V; b0 += 8 * NT) {
      const uint32_t e0 = b0 + 8 * tid;
      float v[8];
      processed(e0, v);
      float p[8];
      uint32_t np = 0, nz = 0, cm = 0;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        p[q] = -1.0f;  // not chosen
        const bool inr = e0 + q < V, fin = inr && v[q] > NEG_INF;
        const bool chosen = fin && bin_of(v[q]) <= last;
        if (fin && !chosen) lkey = umax(lkey, fkey(v[q]));
        if (inr && !fin) p[q] = 0.0f;
        cm |= chosen ? 1u << q : 0u;
      }
      // the exact p of the wave's chosen values, packed in its 256 words of
      // wcnt (free until the sort) so that each lane evaluates about
      // chosen / 64 of them rather than a wave pass per slot holding one
      LDS float* wz = (LDS float*)wcnt + wv * 256;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t hm = (cm >> (4 * h)) & 15u;
        const uint32_t c = (uint32_t)__popc(hm);
        const uint32_t incl = wave_incl_scan(c);
        const uint32_t tot = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
        if (tot == 0) continue;
        uint32_t at = incl - c;
#pragma unroll
        for (int q = 4 * h; q < 4 * h + 4; ++q)
          if ((cm >> q) & 1u) wz[at++] = v[q];
        WaveSync::sync();
        for (uint32_t i = (uint32_t)lane; i < tot; i += WAVE) wz[i] = prob_of(wz[i], P.T, m, S);
        WaveSync::sync();
        at = incl - c;
#pragma unroll
        for (int q = 4 * h; q < 4 * h + 4; ++q)
          if ((cm >> q) & 1u) p[q] = wz[at++];
        WaveSync::sync();
      }
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        if (p[q] > 0.0f) ++np;
        else if (p[q] == 0.0f && !filt) ++nz;
      }
      uint32_t tot;
      const uint32_t off = block_excl_scan(np + (nz << 16), red, tot);
      uint32_t ip = npos + (off & 0xffffu), iz = nzero + (off >> 16);
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        if (p[q] > 0.0f) kA[ip++] = pkey(p[q], e0 + q);
        else if (p[q] == 0.0f && !filt) zl[iz++] = e0 + q;
      }
      npos += tot & 0xffffu;
      nzero += tot >> 16;
    }
    lkey = wave_max_u32(lkey);
    if (lane == 0) red[NW + wv] = lkey;
    wait_stores();
    __syncthreads();
    lkey = 0;
#pragma unroll
    for (int i = 0; i < NW; ++i) lkey = umax(lkey, red[NW + i]);
    const float p_lim = (filt && lkey > 0x007fffffu) ? prob_of(funkey(lkey), P.T, m, S) : 0.0f;
    if (tid == 0) __threadfence();  // drop stale vector-L1 lines before re-reads
    __syncthreads();
    // ---- D: sort, then the semantics
  // stable LSD radix sort of kA[0..npos) on bits 32..63 (kA again holds
  // the sorted keys after its four passes)
  radix_sort_keys(kA, kB, npos, wcnt, digit_off, red);
  GLB uint64_t* src = kA;
    // unpack into p / idx lists (sorted positives, then zeros by index)
    for (uint32_t i = tid; i < npos; i += NT) {
      const uint64_t k = src[i];
      plist[i] = __uint_as_float(~(uint32_t)(k >> 32));
      ilist[i] = (uint32_t)k;
    }
    if (!filt)
      for (uint32_t i = tid; i < nzero; i += NT) {
        plist[npos + i] = 0.0f;
        ilist[npos + i] = zl[i];
      }
    wait_stores();
    __syncthreads();
    if (tid == 0) __threadfence();
    __syncthreads();
    Lst.c = Chain{0.f, 0.f, 0.f, 0};
    // the exact prefix: every entry with p > p_lim (all V when nothing is left out)
    const uint32_t E = filt ? first_below(Lst, npos, p_lim, false, sh + 12) : V;
    const bool good =
        run_semantics<true>(P, u, E, V, p_lim, Lst, sh + 20, (LDS float*)wcnt, tok, len) &&
        !(filt && a.out_cap && len > E && a.out_cap > E);
    if (good && approx) {
      // plist holds the p (= e) unchanged: the slow path's semantics divide
      // through the list's chain
      if (wv == 0) {
        const bool ok = band_certain_wave(ArrAcc<const GLB float*, const GLB uint32_t*>{
                                              plist, ilist},
                                          E, V, p_lim, P.min_p, P.K, P.top_p, u);
        if (tid == 0) sh[9] = ok ? 1u : 0u;
      }
      __syncthreads();
      const bool ok = sh[9] != 0;
      __syncthreads();
      if (!ok) {
        // the reference's S, then the same bins again (chosen by count on a
        // top-k row, whatever S)
        if constexpr (MAT)
          S = exact_normaliser<LLMK_F32>((const float*)proc, nullptr, V, P.T, m, h.bitmap, h.pre,
                                         h.pen, false, smem);
        else
          S = exact_normaliser<DT>(row, mask_row, V, P.T, m, h.bitmap, h.pre, h.pen, true, smem);
        approx = false;
        continue;
      }
    }
    if (good) break;
    last = SLOW_BINS - 1;
    __syncthreads();
  }
  wait_stores();
  __syncthreads();
  write_outputs(a, b, tok, len, Lst, m, S);
  wait_stores();
  __syncthreads();
  if (tid == 0) {
    __threadfence();
    atomicExch(&w.slow_lock[slot], 0u);
  }
  return false;
}

// Key (fkey) of the K-th largest of cval[0..n) (K <= n), by a four-round
// radix select on 8-bit digits.  Every thread of the policy; the digit
// search runs in the policy's first wave.  hist: 256 words, sh: 2 words.
template <class SY>
__device__ __forceinline__ uint32_t kth_largest_key(LDS const float* cval, uint32_t n,
                                                    uint32_t K, LDS uint32_t* hist,
                                                    LDS uint32_t* sh) {
  const uint32_t id = SY::id();
  const int lane = (int)(threadIdx.x & 63);
  uint32_t prefix = 0, need = K;
  for (int round = 0; round < 4; ++round) {
    const int shift = 24 - 8 * round;
    const uint32_t hmask = round == 0 ? 0u : (0xffffffffu << (shift + 8));
    for (uint32_t i = id; i < 256; i += SY::N) hist[i] = 0;
    SY::sync();
    for (uint32_t i = id; i < n; i += SY::N) {
      const uint32_t k = fkey(cval[i]);
      if ((k & hmask) == prefix)
        __atomic_fetch_add(&hist[(k >> shift) & 255u], 1u, __ATOMIC_RELAXED);
    }
    SY::sync();
    if (id < WAVE) {
      // lane l covers digits 255-4l .. 252-4l (descending)
      uint32_t c[4], local = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        c[j] = hist[255 - 4 * lane - j];
        local += c[j];
      }
      const uint32_t incl = wave_incl_scan(local);
      const uint64_t ms = __ballot(incl >= need);
      const int l = __ffsll((unsigned long long)ms) - 1;
      if (lane == l) {
        uint32_t acc = incl - local;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (acc + c[j] >= need) {
            sh[0] = 255u - 4u * (uint32_t)lane - (uint32_t)j;
            sh[1] = need - acc;
            break;
          }
          acc += c[j];
        }
      }
    }
    SY::sync();
    prefix |= sh[0] << shift;
    need = sh[1];
    SY::sync();
  }
  return prefix;
}

// ---------------------------------------------------------------------------
// Finalize one row.  Wave 0 reduces the partials (normaliser S, maximum L)
// and reads the segment table; the candidate path then runs in the whole
// workgroup (a short form when the candidates are in LDS and at most 128
// survive the filter); rows it cannot prove exact take the slow path.
// ---------------------------------------------------------------------------
enum : uint32_t {
  F_DONE = 0, F_S = 1, F_M = 2, F_TOTAL = 3, F_LAM = 4, F_PLIM = 5, F_L = 6, F_GREEDY = 7,
  F_SCR = 8,
  F_BAND = 120  // band_certain_wave's verdict (wave 1 beside wave 0's semantics)
};
// LDS layout of the finalize (words): slots, candidate lists, keys, tables
struct FinLds {
  LDS float* tl;        // MAX_SLOTS: slot maxima
  LDS float* ts;        // MAX_SLOTS: slot sums (or first argmax)
  LDS uint64_t* keys;   // SORT_CAP
  LDS uint64_t* skeys;  // SORT_CAP (sorted)
  LDS float* pp;        // SORT_CAP
  LDS uint32_t* pidx;   // SORT_CAP
  LDS uint32_t* fm;     // 128
  LDS uint32_t* soff;   // MAX_SEG + 16
  LDS uint32_t* red;    // 64
};
__device__ __forceinline__ FinLds fin_carve(LDS uint32_t* smem) {
  FinLds f;
  f.tl = (LDS float*)smem;
  f.ts = f.tl + MAX_SLOTS;
  f.keys = (LDS uint64_t*)(smem + 2 * MAX_SLOTS);
  f.skeys = f.keys + SORT_CAP;
  f.pp = (LDS float*)(f.skeys + SORT_CAP);
  f.pidx = (LDS uint32_t*)(f.pp + SORT_CAP);
  f.fm = f.pidx + SORT_CAP;
  f.soff = f.fm + 128;
  f.red = f.soff + MAX_SEG + 16;
  return f;
}

// Ascending sort of keys[0..n) into skeys[0..n) (keys distinct), by the
// whole workgroup.
//   n <= 256: a rank sort split over the threads (key i against one of
//     NT / npad segments in thread g * npad + i; the partial ranks meet in
//     LDS), three barriers;
//   n <= NT: one key per thread: NT bins over the range of the keys' top
//     words, the keys moved to bin order, then each key's rank among its bin
//     (a key or two, more only for equal probabilities);
//   larger n: a bitonic sort.
// The ranks, bins and moved keys use pp / pidx, free until the sorted keys
// are unpacked.
template <class SY>
__device__ __forceinline__ void sort_keys(const FinLds& f, uint32_t n) {
  if (n <= 256) {
    uint32_t npad = WAVE;
    while (npad < n) npad <<= 1;
    const uint32_t ns = SY::N / npad;
    const uint32_t seg = (n + ns - 1) / ns;
    const uint32_t i = SY::id() % npad, g = SY::id() / npad;
    LDS uint32_t* rk = (LDS uint32_t*)f.pp;
    if (SY::id() < n) rk[SY::id()] = 0;
    SY::sync();
    const uint32_t j0 = g * seg, j1 = umin(j0 + seg, n);
    if (i < n && j0 < j1) {
      const uint64_t k = f.keys[i];
      uint32_t r = 0;
      for (uint32_t j = j0; j < j1; ++j) r += (f.keys[j] < k) ? 1u : 0u;
      if (r) __atomic_fetch_add(&rk[i], r, __ATOMIC_RELAXED);
    }
    SY::sync();
    if (SY::id() < n) f.skeys[rk[SY::id()]] = f.keys[SY::id()];
    SY::sync();
    return;
  }
  if (n <= SY::N) {
    const uint32_t id = SY::id();
    LDS uint64_t* tmp = (LDS uint64_t*)f.pp;  // n keys in bin order
    LDS uint32_t* bo = (LDS uint32_t*)f.pp + 2 * SY::N;  // NT bin offsets
    LDS uint32_t* bq = bo + SY::N;                       // NT cursors
    const uint64_t k = id < n ? f.keys[id] : ~0ull;
    const uint32_t hi = (uint32_t)(k >> 32);
    const uint32_t hmin = block_min_u32(id < n ? hi : EMPTY, f.red);
    const uint32_t hmax = ~block_min_u32(id < n ? ~hi : EMPTY, f.red);
    uint32_t sh = 0;
    while (((hmax - hmin) >> sh) >= SY::N) ++sh;
    const uint32_t bi = (hi - hmin) >> sh;
    bo[id] = 0;
    SY::sync();
    if (id < n) __atomic_fetch_add(&bo[bi], 1u, __ATOMIC_RELAXED);
    SY::sync();
    {
      uint32_t tot;
      const uint32_t ex = block_excl_scan(bo[id], f.red, tot);
      bo[id] = ex;
      bq[id] = ex;
    }
    SY::sync();
    if (id < n) tmp[__atomic_fetch_add(&bq[bi], 1u, __ATOMIC_RELAXED)] = k;
    SY::sync();
    if (id < n) {
      const uint32_t o = bo[bi], oe = bi + 1 < SY::N ? bo[bi + 1] : n;
      uint32_t r = o;
      for (uint32_t j = o; j < oe; ++j) r += tmp[j] < k ? 1u : 0u;
      f.skeys[r] = k;
    }
    SY::sync();
    return;
  }
  uint32_t npad = 1;
  while (npad < n) npad <<= 1;
  for (uint32_t i = SY::id(); i < npad; i += SY::N) f.skeys[i] = i < n ? f.keys[i] : ~0ull;
  SY::sync();
  for (uint32_t k = 2; k <= npad; k <<= 1)
    for (uint32_t j = k >> 1; j > 0; j >>= 1) {
      for (uint32_t i = SY::id(); i < npad / 2; i += SY::N) {
        const uint32_t lo = ((i & ~(j - 1)) << 1) | (i & (j - 1));
        const uint32_t hi = lo | j;
        const uint64_t x = f.skeys[lo], y = f.skeys[hi];
        const bool up = (lo & k) == 0;
        if ((x > y) == up) {
          f.skeys[lo] = y;
          f.skeys[hi] = x;
        }
      }
      SY::sync();
    }
}

// The candidate path under policy SY.  Returns 0 when the row is done, 1
// when its candidates exceed what SY handles, 2 when it needs the slow path,
// 4 when a row sampled with S = 1 (approx) cannot be proven by the band
// check (the reference's S is needed).
template <class SY>
__device__ __forceinline__ uint32_t candidate_path(const Args& a, const Ws& w, uint32_t b,
                                                   const RowP& P, float S, float m, float u,
                                                   uint32_t total, uint32_t lam,
                                                   const FinLds& f, uint32_t gather_cap,
                                                   uint32_t keep_cap, bool approx) {
  LDS const u2v* lcand = (LDS const u2v*)((LDS uint32_t*)f.tl + a.lds_cand);
  const uint32_t id = SY::id();
  if (total > gather_cap) return 1;
  const bool topk = P.K > 0 && (uint32_t)P.K < a.V;
  const float plim = __uint_as_float(f.fm[F_PLIM]);
  uint32_t lam_e = lam;
  float plim_e = plim;
  constexpr int GQ = 8;  // candidate loads in flight per thread
  // candidate i of the row: the LDS list, else the segments' global buffers
  auto load = [&](uint32_t i) __attribute__((always_inline)) {
    u2v e = u2v{0xff800000u, 0u};
    if (i < total && a.G == 1 && i < LCAP) {
      e = lcand[i];
    } else if (i < total) {
      uint32_t lo = 0, hi = a.G;  // soff[lo] <= i < soff[hi]
      while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) >> 1;
        if (f.soff[mid] <= i) lo = mid;
        else hi = mid;
      }
      e = G(w.cand)[(uint64_t)row_seg_to_wg(a, b, lo) * CAND_CAP + (i - f.soff[lo])];
    }
    return e;
  };
  // Probability bins: the exact p of a candidate above plim falls in a bin
  // of its top bits (exponent and 4 mantissa bits, 2033 bins for p <= 1),
  // with its count and mass.  The kept set is the bins from the top down to
  // the first that brings the count to K (top-k rows) or the mass to top_p
  // (the uniform when top-p is off) + 0.002; entries below the last kept
  // bin then have p below its lower edge.  The bins live in skeys, free
  // until the kept keys are sorted.
  LDS uint32_t* bcnt = (LDS uint32_t*)f.skeys;
  LDS float* bmass = (LDS float*)f.skeys + 2048;
  auto hist_clear = [&]() __attribute__((always_inline)) {
    for (uint32_t i = id; i < 2048; i += SY::N) {
      bcnt[i] = 0;
      bmass[i] = 0.0f;
    }
    if (id == 0) f.fm[F_SCR + 2] = 0;
  };
  // the largest binned p: a running maximum per thread, one atomic per wave
  // after the pass (an atomic per candidate on one word serialises)
  uint32_t pmx = 0;
  auto hist_add = [&](float pv) __attribute__((always_inline)) {
    const uint32_t bi = __float_as_uint(pv) >> 19;
    __atomic_fetch_add(&bcnt[bi], 1u, __ATOMIC_RELAXED);
    __atomic_fetch_add(&bmass[bi], pv, __ATOMIC_RELAXED);
    pmx = umax(pmx, __float_as_uint(pv));
  };
  auto hist_flush = [&]() __attribute__((always_inline)) {
    const uint32_t x = wave_max_u32(pmx);
    if ((id & 63u) == 0 && x) __atomic_fetch_max(&f.fm[F_SCR + 2], x, __ATOMIC_RELAXED);
    pmx = 0;
  };
  // pv of candidate e if it is at or above lam (0 otherwise), where a lane
  // of the wave needs one
  auto exact_p = [&](u2v e, bool& g) __attribute__((always_inline)) {
    const float v = __uint_as_float(e.x);
    g = v > NEG_INF && fkey(v) >= lam;
    float pv = 0.0f;
    if (__ballot(g) != 0 && g) pv = prob_of(v, P.T, m, S);
    return pv;
  };
  // a further pass over the candidates from their buffers: fn(kept, p, idx)
  auto each = [&](auto&& fn) __attribute__((always_inline)) {
    for (uint32_t i0 = 0; i0 < total; i0 += GQ * SY::N) {
      u2v e[GQ];
#pragma unroll
      for (int q = 0; q < GQ; ++q) e[q] = load(i0 + q * SY::N + id);
#pragma unroll
      for (int q = 0; q < GQ; ++q) {
        if (i0 + q * SY::N >= total) break;
        bool g;
        const float pv = exact_p(e[q], g);
        fn(g && pv > plim, pv, e[q].y);
      }
    }
  };
  // ---- one pass over the candidates at or above lam (every element not in
  // the buffers has a key below lam): top-k rows keep (logit, idx), other
  // rows (p, idx) of those with p > plim, binned; one scan per GQ slots
  LDS float* cval = f.pp;
  LDS uint32_t* cidx = f.pidx;
  if (!topk) {
    hist_clear();
    SY::sync();
  }
  uint32_t n0 = 0;
  for (uint32_t i0 = 0; i0 < total; i0 += GQ * SY::N) {
    u2v e[GQ];
#pragma unroll
    for (int q = 0; q < GQ; ++q) e[q] = load(i0 + q * SY::N + id);
    float val[GQ];
    uint32_t km = 0;
#pragma unroll
    for (int q = 0; q < GQ; ++q) {
      if (topk) {
        const float v = __uint_as_float(e[q].x);
        val[q] = v;
        if (v > NEG_INF && fkey(v) >= lam) km |= 1u << q;
      } else {
        bool g;
        val[q] = exact_p(e[q], g);
        if (g && val[q] > plim) {
          km |= 1u << q;
          hist_add(val[q]);
        }
      }
    }
    uint32_t tot;
    uint32_t pos = n0 + block_excl_scan((uint32_t)__popc(km), f.red, tot);
#pragma unroll
    for (int q = 0; q < GQ; ++q)
      if ((km >> q) & 1u) {
        if (pos < SORT_CAP) {
          cval[pos] = val[q];
          cidx[pos] = e[q].y;
        }
        ++pos;
      }
    n0 += tot;
  }
  if (!topk) hist_flush();
  SY::sync();
  // ---- min-p first (top-k rows): an entry below fl(min_p * p_max) is cut
  // by the semantics' first step and never read after it, so the gathered
  // entries below it are dropped now, in order; the largest dropped p then
  // bounds everything past the list from below the threshold, which tells
  // the semantics that the cut lies at the list's end.
  float pdrop = 0.0f;
  if (topk && P.min_p > 0.0f && n0 <= SORT_CAP) {
    float pm = 0.0f;
    for (uint32_t i = id; i < n0; i += SY::N) pm = fmaxf(pm, prob_of(cval[i], P.T, m, S));
    pm = block_max(pm, (LDS float*)f.red);
    const float t = P.min_p * pm;
    uint32_t nk = 0;
    for (uint32_t i0 = 0; i0 < n0; i0 += SY::N) {
      const uint32_t i = i0 + id;
      float v = 0.0f;
      uint32_t ix = 0;
      bool keep = false;
      if (i < n0) {
        v = cval[i];
        ix = cidx[i];
        const float pv = prob_of(v, P.T, m, S);
        keep = pv >= t;
        if (!keep) pdrop = fmaxf(pdrop, pv);
      }
      // every read of this round precedes the scan's barriers; the writes
      // land below the next round's entries
      uint32_t tot;
      const uint32_t pos = nk + SY::excl_scan(keep, f.red, tot);
      if (keep) {
        cval[pos] = v;
        cidx[pos] = ix;
      }
      nk += tot;
    }
    pdrop = block_max(pdrop, (LDS float*)f.red);
    n0 = nk;
  }
  uint32_t n = 0;
  if (!topk || n0 > SORT_CAP) {
    if (topk) {
      // more than SORT_CAP top-k candidates: bin them by p, a second pass
      hist_clear();
      SY::sync();
      each([&](bool k, float pv, uint32_t) __attribute__((always_inline)) {
        if (k) hist_add(pv);
      });
      hist_flush();
      SY::sync();
    }
    if (threadIdx.x < WAVE) {
      // lane l: bins 2047 - 32 l down to 2016 - 32 l
      const int lane = (int)threadIdx.x;
      const float tm = (P.top_p < 1.0f ? P.top_p : u) + 0.002f;
      const bool use_mass = !topk && tm < 1.0f;
      uint32_t c = 0;
      float ms = 0.0f;
      for (int k = 0; k < 32; ++k) {
        const uint32_t bi = 2047u - 32u * (uint32_t)lane - (uint32_t)k;
        c += bcnt[bi];
        ms += bmass[bi];
      }
      const uint32_t cincl = wave_incl_scan(c);
      float mincl = ms;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const float o = __shfl_up(mincl, d);
        if (lane >= d) mincl += o;
      }
      const uint64_t hit = topk ? __ballot(cincl >= (uint32_t)P.K)
                                : (use_mass ? __ballot(mincl >= tm) : 0ull);
      uint32_t tb = 0;  // the last kept bin (0: every bin)
      if (hit) {
        const int l = __ffsll((unsigned long long)hit) - 1;
        uint32_t cc = (uint32_t)__shfl((int)(cincl - c), l);
        float mm = __shfl(mincl - ms, l);
        for (int k = 0; k < 32; ++k) {
          const uint32_t bi = 2047u - 32u * (uint32_t)l - (uint32_t)k;
          cc += bcnt[bi];
          mm += bmass[bi];
          if (topk ? cc >= (uint32_t)P.K : mm >= tm) {
            tb = bi;
            break;
          }
        }
      }
      // min-p: the semantics' first step keeps p >= min_p * p_max and
      // renormalises by the sum of exactly those, and every later step reads
      // only them, so the kept bins are those down to the one below the
      // threshold's (its cut seen, or lying past every kept entry) whatever
      // the count or mass rule asks
      if (P.min_p > 0.0f) {
        const uint32_t tk = __float_as_uint(P.min_p * __uint_as_float(f.fm[F_SCR + 2])) >> 19;
        tb = tk > 0 ? tk - 1 : 0u;
      }
      uint32_t nk = 0;
      for (uint32_t k = (uint32_t)lane; k < 2048; k += WAVE) nk += k >= tb ? bcnt[k] : 0u;
      nk = bcast63u(wave_incl_scan(nk));
      if (lane == 0) {
        f.fm[F_SCR] = tb;
        f.fm[F_SCR + 1] = nk;
      }
    }
    SY::sync();
    const uint32_t tb = f.fm[F_SCR], nk = f.fm[F_SCR + 1];
    SY::sync();
    if (nk > SORT_CAP) return 2;
    const uint32_t tbits = tb << 19;
    if (tbits > 0) plim_e = fmaxf(plim, __uint_as_float(tbits - 1));
    if (!topk && n0 <= SORT_CAP) {
      // the kept bins, from the gathered (p, idx) in LDS
      for (uint32_t i0 = 0; i0 < n0; i0 += SY::N) {
        const uint32_t i = i0 + id;
        const bool keep = i < n0 && __float_as_uint(cval[i]) >= tbits;
        uint32_t tot;
        const uint32_t pos = n + SY::excl_scan(keep, f.red, tot);
        if (keep) f.keys[pos] = pkey(cval[i], cidx[i]);
        n += tot;
      }
    } else {
      each([&](bool k, float pv, uint32_t ix) __attribute__((always_inline)) {
        const bool keep = k && __float_as_uint(pv) >= tbits;
        uint32_t tot;
        const uint32_t pos = n + SY::excl_scan(keep, f.red, tot);
        if (keep) f.keys[pos] = pkey(pv, ix);
        n += tot;
      });
    }
  } else {
  // ---- top-k rows: the exact (K+1)-th largest candidate logit tightens
  // the bound (every element below it has p <= plim of that bound; the
  // entry past the K-th stays in the list for the band check)
  if (n0 > 2u * (uint32_t)P.K) {
    const uint32_t tau = kth_largest_key<SY>(cval, n0, (uint32_t)P.K + 1u,
                                             (LDS uint32_t*)f.keys, f.fm + F_SCR);
    lam_e = tau;
    plim_e = tau > 0x007fffffu ? prob_of(funkey(tau - 1), P.T, m, S) : 0.0f;
  }
  for (int attempt = 0; attempt < 2; ++attempt) {
    n = 0;
    for (uint32_t i0 = 0; i0 < n0; i0 += SY::N) {
      const uint32_t i = i0 + id;
      bool keep = false;
      uint64_t key = 0;
      if (i < n0) {
        const float v = cval[i];
        if (fkey(v) >= lam_e) {
          const float pv = prob_of(v, P.T, m, S);
          if (pv > plim_e) {
            keep = true;
            key = pkey(pv, cidx[i]);
          }
        }
      }
      uint32_t tot;
      const uint32_t pos = n + SY::excl_scan(keep, f.red, tot);
      if (keep) f.keys[pos] = key;
      n += tot;
    }
    // a tightened bound that keeps fewer than K + 1 (ties in p across it)
    // falls back to the gather bound
    if (!(topk && n < (uint32_t)P.K + 1u && lam_e != lam)) break;
    lam_e = lam;
    plim_e = plim;
  }
  }
  SY::sync();
  plim_e = fmaxf(plim_e, pdrop);  // also bounds the entries min-p dropped
  if (n > keep_cap) return 1;
  sort_keys<SY>(f, n);
  for (uint32_t i = id; i < n; i += SY::N) {
    const uint64_t k = f.skeys[i];
    f.pp[i] = __uint_as_float(~(uint32_t)(k >> 32));
    f.pidx[i] = (uint32_t)k;
  }
  SY::sync();
  // ---- min-p / top-k / top-p / draw in wave 0 (and the band check of a
  // row sampled with S = 1 in wave 1 beside it, or after a workgroup's
  // semantics); outputs only once the result stands
  uint32_t res = 2;
  if (n <= 128) {
    float p0 = 0.0f, p1 = 0.0f;
    uint32_t i0 = 0, i1 = 0, tok = 0, len = 0;
    bool good = false;
    if (threadIdx.x < WAVE) {
      const int lane = (int)threadIdx.x;
      p0 = (uint32_t)lane < n ? f.pp[lane] : 0.0f;
      p1 = (uint32_t)lane + 64 < n ? f.pp[64 + lane] : 0.0f;
      i0 = (uint32_t)lane < n ? f.pidx[lane] : 0u;
      i1 = (uint32_t)lane + 64 < n ? f.pidx[64 + lane] : 0u;
      // f.keys is free once sorted into skeys and copied out
      good = semantics_regs(P, u, n, a.V, plim_e, p0, p1, i0, i1, lane,
                            (LDS float*)f.keys, tok, len);
      if (good && a.out_cap && len > n && a.out_cap > n) good = false;
    } else if (approx && threadIdx.x < 2 * WAVE) {
      const bool ok = band_certain_wave(KeyAcc{f.skeys}, n, a.V, plim_e, P.min_p, P.K,
                                        P.top_p, u);
      if (threadIdx.x == WAVE) f.fm[F_BAND] = ok ? 1u : 0u;
    }
    if (approx) SY::sync();
    if (threadIdx.x < WAVE) {
      const int lane = (int)threadIdx.x;
      if (good && approx && f.fm[F_BAND] == 0) {
        good = false;
        res = 4;
      } else {
        res = good ? 0u : 2u;
      }
      if (good) {
        const uint32_t ic = a.cut ? cut_id(len, n, i0, i1) : 0u;
        if (lane == 0) {
          G(a.out_tok)[b] = tok;
          if (a.out_cnt) G(a.out_cnt)[b] = len;
          if (a.cut) G(a.cut)[b] = u4v{ic, len, __float_as_uint(m), __float_as_uint(S)};
        }
        const uint32_t no = len < a.out_cap ? len : a.out_cap;
        const uint64_t ob = (uint64_t)b * a.out_cap;
        if ((uint32_t)lane < no) {
          if (a.out_ids) G(a.out_ids)[ob + lane] = i0;
          if (a.out_probs) G(a.out_probs)[ob + lane] = p0;
        }
        if ((uint32_t)lane + 64 < no) {
          if (a.out_ids) G(a.out_ids)[ob + 64 + lane] = i1;
          if (a.out_probs) G(a.out_probs)[ob + 64 + lane] = p1;
        }
      }
    }
  } else {
    List Ls{flat(f.pp), flat(f.pidx), Chain{0.f, 0.f, 0.f, 0}, (float*)f.pp};
    uint32_t tok = 0, len = 0;
    bool good = run_semantics<false>(P, u, n, a.V, plim_e, Ls, f.fm + F_SCR,
                                     (LDS float*)f.keys, tok, len);
    if (good && a.out_cap && len > n && a.out_cap > n) good = false;
    res = good ? 0u : 2u;
    if (good && approx) {
      // the sorted keys are intact (the semantics divided pp in place)
      if (threadIdx.x < WAVE) {
        const bool ok = band_certain_wave(KeyAcc{f.skeys}, n, a.V, plim_e, P.min_p, P.K,
                                          P.top_p, u);
        if (threadIdx.x == 0) f.fm[F_BAND] = ok ? 1u : 0u;
      }
      SY::sync();
      if (f.fm[F_BAND] == 0) {
        good = false;
        res = 4;
      }
    }
    if (good) write_outputs(a, b, tok, len, Ls, m, S);
  }
  if (SY::N > WAVE) {
    if (threadIdx.x == 0) f.fm[F_DONE] = res;
    SY::sync();
    res = f.fm[F_DONE];
  }
  return res;
}

// The candidate path of a single-segment row whose candidates are all in
// LDS (total <= LCAP), with the whole workgroup: one candidate per thread
// for the gather and the filter, the rank sort split eight ways (each
// thread compares one key with sixteen others), the semantics in wave 0
// from registers, and on a row sampled with S = 1 (approx) the band check
// in wave 1 beside them.  Returns 0 when the row is done, 1 when it needs
// the general path (more than 128 kept), 2 for the slow path, 4 when S = 1
// cannot be proven (the reference's S is needed).
__device__ __forceinline__ uint32_t candidate_fast(const Args& a, uint32_t b, const RowP& P,
                                                   float S, float m, float u, uint32_t total,
                                                   uint32_t lam, const FinLds& f, bool approx) {
  using SY = BlockSync;
  const uint32_t tid = threadIdx.x;
  LDS const u2v* lcand = (LDS const u2v*)((LDS uint32_t*)f.tl + a.lds_cand);
  LDS float* cval = f.pp;
  LDS uint32_t* cidx = f.pidx;
  // ---- gather the candidates at or above lam, and in the same pass their
  // exact probabilities above the bound as (p desc, idx asc) keys; one scan
  // counts both (packed in 16-bit halves: total <= LCAP)
  const bool topk = P.K > 0 && (uint32_t)P.K < a.V;
  const float plim = __uint_as_float(f.fm[F_PLIM]);
  const u2v e = tid < total ? lcand[tid] : u2v{0xff800000u, 0u};
  const float v0 = __uint_as_float(e.x);
  const bool g0 = v0 > NEG_INF && fkey(v0) >= lam;
  const float pv0 = g0 ? prob_of(v0, P.T, m, S) : 0.0f;
  const bool k0 = g0 && pv0 > plim;
  uint32_t both;
  const uint32_t pos = block_excl_scan((g0 ? 1u : 0u) + (k0 ? 0x10000u : 0u), f.red, both);
  const uint32_t n0 = both & 0xffffu;
  uint32_t n = both >> 16;
  float ptail = plim;  // every element not kept has p <= ptail
  // the kept list reaches one entry past the K-th, which the band check
  // compares with the K-th
  const uint32_t K1 = topk ? umin((uint32_t)P.K + 1u, n0) : 0u;
  if (n <= 128 || !topk) {
    if (k0) f.keys[pos >> 16] = pkey(pv0, e.y);
  } else {
    // more than 128 kept: the exact (K+1)-th largest tightens the bound
    if (g0) {
      cval[pos & 0xffffu] = v0;
      cidx[pos & 0xffffu] = e.y;
    }
    SY::sync();
    const uint32_t tau = kth_largest_key<SY>(cval, n0, K1, (LDS uint32_t*)f.keys,
                                             f.fm + F_SCR);
    uint32_t lam_e = tau;
    float plim_e = tau > 0x007fffffu ? prob_of(funkey(tau - 1), P.T, m, S) : 0.0f;
    for (int attempt = 0; attempt < 2; ++attempt) {
      bool keep = false;
      uint64_t key = 0;
      if (tid < n0) {
        const float v = cval[tid];
        if (fkey(v) >= lam_e) {
          const float pv = prob_of(v, P.T, m, S);
          if (pv > plim_e) {
            keep = true;
            key = pkey(pv, cidx[tid]);
          }
        }
      }
      const uint32_t p2 = SY::excl_scan(keep, f.red, n);
      if (keep) f.keys[p2] = key;
      // a tightened bound that keeps fewer than K + 1 (ties in p across it)
      // falls back to the gather bound
      if (!(n < K1 && lam_e != lam)) break;
      lam_e = lam;
      plim_e = plim;
    }
    ptail = plim_e;
  }
  if (n > 128) return 1;
  // ---- rank sort: key i against keys 16s .. 16s+15 in thread 128s + i
  LDS uint32_t* rk = (LDS uint32_t*)cval;  // 128 ranks; cval is read no more
  if (tid < 128) rk[tid] = 0;
  SY::sync();
  {
    const uint32_t i = tid & 127u, s0 = 16u * (tid >> 7);
    if (i < n && s0 < n) {
      const uint64_t k = f.keys[i];
      uint64_t x[16];
#pragma unroll
      for (uint32_t e = 0; e < 16; ++e) x[e] = (s0 + e < n) ? f.keys[s0 + e] : ~0ull;
      uint32_t r = 0;
#pragma unroll
      for (uint32_t e = 0; e < 16; ++e) r += (x[e] < k) ? 1u : 0u;
      if (r) __atomic_fetch_add(&rk[i], r, __ATOMIC_RELAXED);
    }
  }
  SY::sync();
  if (tid < n) f.skeys[rk[tid]] = f.keys[tid];
  SY::sync();
  // ---- min-p / top-k / top-p / draw in wave 0; the outputs are written
  // after the barrier that publishes the result, which then waits for no
  // global store
  float p0 = 0.0f, p1 = 0.0f;
  uint32_t i0 = 0, i1 = 0, tok = 0, len = 0;
  bool good = false;
  if (tid < WAVE) {
    const int lane = (int)tid;
    const uint64_t k0 = (uint32_t)lane < n ? f.skeys[lane] : 0ull;
    const uint64_t k1 = (uint32_t)lane + 64 < n ? f.skeys[64 + lane] : 0ull;
    p0 = (uint32_t)lane < n ? __uint_as_float(~(uint32_t)(k0 >> 32)) : 0.0f;
    p1 = (uint32_t)lane + 64 < n ? __uint_as_float(~(uint32_t)(k1 >> 32)) : 0.0f;
    i0 = (uint32_t)k0;
    i1 = (uint32_t)k1;
    // f.keys is free once sorted into skeys
    good = semantics_regs(P, u, n, a.V, ptail, p0, p1, i0, i1, lane, (LDS float*)f.keys, tok,
                          len);
    if (good && a.out_cap && len > n && a.out_cap > n) good = false;
    if (lane == 0) f.fm[F_DONE] = good ? 0u : 2u;
  } else if (approx && tid < 2 * WAVE) {
    const bool ok = band_certain_wave(KeyAcc{f.skeys}, n, a.V, ptail, P.min_p, P.K, P.top_p, u);
    if (tid == WAVE) f.fm[F_BAND] = ok ? 1u : 0u;
  }
  SY::sync();
  uint32_t res = f.fm[F_DONE];
  if (res == 0 && approx && f.fm[F_BAND] == 0) res = 4;
  if (tid < WAVE && res == 0) {
    const int lane = (int)tid;
    const uint32_t ic = a.cut ? cut_id(len, n, i0, i1) : 0u;
    if (lane == 0) {
      G(a.out_tok)[b] = tok;
      if (a.out_cnt) G(a.out_cnt)[b] = len;
      if (a.cut) G(a.cut)[b] = u4v{ic, len, __float_as_uint(m), __float_as_uint(S)};
    }
    const uint32_t no = len < a.out_cap ? len : a.out_cap;
    const uint64_t ob = (uint64_t)b * a.out_cap;
    if ((uint32_t)lane < no) {
      if (a.out_ids) G(a.out_ids)[ob + lane] = i0;
      if (a.out_probs) G(a.out_probs)[ob + lane] = p0;
    }
    if ((uint32_t)lane + 64 < no) {
      if (a.out_ids) G(a.out_ids)[ob + 64 + lane] = i1;
      if (a.out_probs) G(a.out_probs)[ob + 64 + lane] = p1;
    }
  }
  return res;
}

// ---------------------------------------------------------------------------
// The kernel's arguments for a call of its own
// ---------------------------------------------------------------------------
// A rare path made a call of its own, so that its registers are allocated
// apart from the stream path's (inlined together, they spilled), reads the
// kernel's arguments from the copy in g_kctx, which the kernel writes
// before the call (passed by reference, they would be copied to scratch).
struct KCtx {
  Args a;
  Ws w;
};
__shared__ KCtx g_kctx;
// stream_kernel's parameters lie in the kernel-argument segment in order,
// each at its natural alignment: a at 0, w next, as in KCtx.
constexpr size_t kWsOffset = (sizeof(Args) + alignof(Ws) - 1) / alignof(Ws) * alignof(Ws);
static_assert(offsetof(KCtx, w) == kWsOffset, "KCtx mirrors the kernel's parameters");
// Copies the kernel's parameters into g_kctx, a word a thread from the
// kernel-argument segment (copying the by-value parameters instead would
// keep every field of them in registers from the kernel's start).  In a
// kernel only; every thread, a barrier after it.
__device__ __forceinline__ void kctx_fill() {
  typedef const __attribute__((address_space(4))) uint32_t KWord;
  KWord* k = (KWord*)__builtin_amdgcn_kernarg_segment_ptr();
  LDS uint32_t* d = (LDS uint32_t*)&g_kctx;
  for (uint32_t i = threadIdx.x; i < (uint32_t)(sizeof(KCtx) / 4); i += NT) d[i] = k[i];
}
// The arguments back from g_kctx into scalar registers: every word is
// the same in all lanes, which a read of the first lane tells the compiler
// (loaded as they are, each would take a vector register).
__device__ __forceinline__ KCtx kctx_load() {
  constexpr uint32_t N = (uint32_t)(sizeof(KCtx) / 4);
  uint32_t wd[N];
#pragma unroll
  for (uint32_t i = 0; i < N; ++i)
    wd[i] = (uint32_t)__builtin_amdgcn_readfirstlane((int)((LDS const uint32_t*)&g_kctx)[i]);
  KCtx c;
  __builtin_memcpy(&c, wd, sizeof(KCtx));
  return c;
}

// The segment table (counts, thresholds, flags of the row's segments), the
// bound plim, then the candidate path: 0 when the row is done, 2 for the
// slow path, 4 when approx (S = 1) could not be proven, 5 when a segment's
// history (or, hist_ovf, the whole row's) outgrew the LDS tables.  Every
// thread.
template <int DT>
__device__ __forceinline__ uint32_t candidate_paths(const Args& a, const Ws& w, uint32_t b,
                                                    const RowP& P, float S, float m, float L,
                                                    float u, u4v seg_own, bool approx,
                                                    LDS uint32_t* smem, bool hist_ovf = false) {
  const uint32_t tid = threadIdx.x;
  const int lane = (int)(tid & 63), wv = (int)(tid >> 6);
  const FinLds f = fin_carve(smem);
  uint32_t path = 2;  // 0 done, 1 workgroup candidate path, 2 slow path, 3 fast path
  if (wv == 0) {
    // ---- segment table: counts, thresholds, flags
    uint32_t cnt = 0, beta = 0, flg = 0;
    if (a.G == 1) {
      if (lane == 0) {
        cnt = seg_own.x < CAND_CAP ? seg_own.x : CAND_CAP;
        beta = seg_own.y;
        flg = seg_own.z;
      }
    } else if ((uint32_t)lane < a.G) {
      const u4v sm = G(w.seg_meta)[row_seg_to_wg(a, b, (uint32_t)lane)];
      cnt = sm.x < CAND_CAP ? sm.x : CAND_CAP;
      beta = sm.y;
      flg = sm.z;
    }
    const uint32_t lam = wave_max_u32(beta << BIN_SHIFT);
    const bool ovf = __ballot((flg & FLAG_OVERFLOW) != 0) != 0;
    const uint32_t off_incl = wave_incl_scan(cnt);
    const uint32_t total = bcast63u(off_incl);
    if ((uint32_t)lane <= a.G) f.soff[lane] = off_incl - cnt;  // lane G: the total
    WaveSync::sync();
    // the bound on p of every element outside the candidate buffers, once
    // (wave 0) rather than in every thread of the candidate path
    const float plim = lam > 0x007fffffu ? prob_of(funkey(lam - 1), P.T, m, S) : 0.0f;
    if (lane == 0) {
      f.fm[F_S] = __float_as_uint(S);
      f.fm[F_M] = __float_as_uint(m);
      f.fm[F_L] = __float_as_uint(L);
      f.fm[F_PLIM] = __float_as_uint(plim);
      f.fm[F_TOTAL] = total;
      f.fm[F_LAM] = lam;
    }
    if (!(L == NEG_INF || P.Kc == 0 || ovf))
      path = (a.G == 1 && total <= LCAP) ? 3u : 1u;
    if (hist_ovf || __ballot((flg & FLAG_HIST_OVERFLOW) != 0) != 0ull) path = 5;
    if (lane == 0) f.fm[F_DONE] = path;
  }
  __syncthreads();
  path = f.fm[F_DONE];
  if (path == 3) {
    path = candidate_fast(a, b, P, S, m, u, f.fm[F_TOTAL], f.fm[F_LAM], f, approx);
    if (path == 0) return 0;
  }
  if (path == 1) {
    const uint32_t total = f.fm[F_TOTAL], lam = f.fm[F_LAM];
    __syncthreads();
    path = candidate_path<BlockSync>(a, w, b, P, S, m, u, total, lam, f, EMPTY, SORT_CAP,
                                     approx);
    if (path == 0) return 0;
  }
  __syncthreads();
  return path;
}

// The slow path over the materialised row (slow_row<DT, true>): a call of
// its own, so that the other rare paths keep their registers; the kernel's
// arguments from g_kctx.
template <int DT>
__device__ __noinline__ void slow_row_mat(uint32_t b, RowP P, bool approx, bool need_exact) {
  extern __shared__ __align__(16) uint32_t smem[];
  const KCtx c = kctx_load();
  (void)slow_row<DT, true>(c.a, c.w, b, P, approx ? 1.0f : 0.0f, 0.0f, 0.0f,
                           (LDS uint32_t*)smem, approx, need_exact);
}

// Path 4 of finalize_rare: the reference's S (S_in when it is given, not
// NaN, as the many-workgroup sum of phase 1 hands it over), then the
// candidate path again (or the slow path).  Returns true when the row's
// history outgrows the tables (the materialised slow path then takes it).
template <int DT>
__device__ __forceinline__ bool exact_rerun(const Args& a, const Ws& w, uint32_t b,
                                            const RowP& P, float m, float L, float u,
                                            u4v seg_own, LDS uint32_t* sm, float S_in) {
  const uint32_t tid = threadIdx.x;
  LDS uint32_t* sc = sm;  // below the tables in both layouts
  const void* row = (const char*)a.logits +
                    (uint64_t)b * a.stride * ((DT & 3) == LLMK_F32 ? 4u : 2u);
  // a single-segment row's tables where its stream phase had them (below
  // its kept partials and candidates, which the candidate path reads again);
  // a row of several segments in the slow path's layout
  Hist h;
  const uint32_t nwords = a.G == 1 ? a.ntiles * 32 : (a.V + 31) / 32;
  hist_carve(h, a.G == 1 ? sm + 64 + M_NMISC + NBINS + 64 : sm + 128 + 256 + NW * 256 + SLOW_BINS,
             nwords);
  h.lo = 0;
  // The tables serve the normaliser and tell whether the whole row's history
  // outgrows them.  With S given, a single-segment row needs neither: its
  // one segment's tables held the whole row's history without overflow.
  if (!(S_in == S_in && a.G == 1)) {
    if (tid == 0) sc[64] = 0;
    build_history<DT>(a, P, b, row, 0, a.V, nwords, h, sc + 128, &sc[64]);
    if (sc[64] & FLAG_HIST_OVERFLOW) return true;  // the whole row's history outgrows them
  }
  const float S =
      S_in == S_in
          ? S_in
          : exact_normaliser<DT>(row, a.mask ? a.mask + (uint64_t)b * a.mask_words : nullptr,
                                 a.V, P.T, m, h.bitmap, h.pre, h.pen, true, sc);
  __syncthreads();
  const uint32_t path = candidate_paths<DT>(a, w, b, P, S, m, L, u, seg_own, false, sm);
  return path != 0 && slow_row<DT, false>(a, w, b, P, S, m, L, sm, false, false);
}

// Posts a row whose band check failed as a job of phase 1 (the launch after
// this one sums its S on many workgroups and finishes the row): its
// parameters, m, L, u, seg_own and, for a single-segment row, the LDS
// partials and candidates the candidate path reads again.  False when the
// call's xs_cap jobs are taken (the row is then finished here).
__device__ __forceinline__ bool xs_post(const Args& a, const Ws& w, uint32_t b, const RowP& P,
                                        float m, float L, float u, u4v seg_own,
                                        LDS uint32_t* sm) {
  const uint32_t tid = threadIdx.x;
  if (a.xs_cap == 0) return false;  // no phase 1 in this call
  if (tid == 0)
    g_bcast[2] = __hip_atomic_fetch_add(&w.xs_ctl[a.epoch & 1u], 1u, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  const uint32_t j = g_bcast[2];
  if (j >= a.xs_cap) return false;
  GLB uint32_t* rec = G(w.xs_job) + (uint64_t)j * XS_JOB_WORDS;
  if (tid == 0) {
    rec[0] = b;
    rec[1] = __float_as_uint(P.T);
    rec[2] = __float_as_uint(P.top_p);
    rec[3] = __float_as_uint(P.min_p);
    rec[4] = __float_as_uint(P.rp);
    rec[5] = __float_as_uint(P.pp);
    rec[6] = __float_as_uint(P.fp);
    rec[7] = (uint32_t)P.K;
    rec[8] = P.mode;
    rec[9] = P.Kc;
    rec[10] = __float_as_uint(m);
    rec[11] = __float_as_uint(L);
    rec[12] = __float_as_uint(u);
    rec[13] = seg_own.x;
    rec[14] = seg_own.y;
    rec[15] = seg_own.z;
    rec[16] = seg_own.w;
  }
  if (a.G == 1) {
    GLB uint32_t* sv = G(w.xs_save) + (uint64_t)j * XS_SAVE;
    for (uint32_t i = tid; i < XS_SAVE; i += NT) sv[i] = sm[a.lds_part + i];
  }
  return true;  // the kernel's end orders these stores before phase 1
}

// The rows the candidate path did not finish (path: 2, the slow path; 4, a
// row that top-k renormalises whose band check failed; 5, a row whose
// history outgrows the LDS tables, which the slow path materialises, with
// approx for a row that top-k renormalises; 6, a row of path 4 back from
// phase 1 with the reference's S).  For path 4 the reference's S
// (exact_normaliser, over the row's history tables, built again: the
// candidate path has overwritten a single-segment row's own), then the
// candidate path again in the reference's arithmetic, else the slow path.
// A call of its own (rare), its registers allocated apart from the stream
// path's; it reads the kernel's arguments from g_kctx, which the caller
// writes first.  The materialised slow path is one call at its end (a call
// in each branch cost the others registers: apply_top_p 470 -> 525 us).
template <int DT>
__device__ __noinline__ void finalize_rare(uint32_t b, RowP P, float S, float m, float L,
                                           float u, u4v seg_own, bool approx, uint32_t path) {
  extern __shared__ __align__(16) uint32_t smem[];
  const KCtx c = kctx_load();
  const Args& a = c.a;
  const Ws& w = c.w;
  LDS uint32_t* sm = (LDS uint32_t*)smem;
  // mat: the row goes to the materialised slow path (one call, at the end)
  bool mat = path == 5;
  if (!mat && path != 4 && path != 6) {
    mat = slow_row<DT, false>(a, w, b, P, S, m, L, sm, approx, false);
  } else if (!mat) {
    if (path == 4 && a.phase == 0 && xs_post(a, w, b, P, m, L, u, seg_own, sm)) return;
    mat = exact_rerun<DT>(a, w, b, P, m, L, u, seg_own, sm, path == 6 ? S : __builtin_nanf(""));
    approx = false;
  }
  if (mat) slow_row_mat<DT>(b, P, approx, !approx);
}

// ---------------------------------------------------------------------------
// Phase 1: the reference's S of the rows whose band check failed, on many
// workgroups
// ---------------------------------------------------------------------------
// The launch after the sampling launch, grid xs_cap x nwin: workgroup (j, k)
// takes window k (XS_W elements) of job j's row; the last window of a job
// to finish walks the windows and finishes the row.  A window:
//   * its processed logits (history tables of its own range, the mask) and
//     the exact terms e = exp_ref(fl(l / T) - m) of all its elements, whose
//     f32 sum A_k it publishes (release) for the windows after it;
//   * the sums of the windows before it (acquire; they run beside it: the
//     grid fits the GPU, one workgroup a CU, and a wait that runs out drops
//     only the estimate) give the exact sequential sum at its start c_k to
//     within a relative (window end) n u: recursive f32 summation of
//     positive terms is off by at most u per addition of the sum so far,
//     and each A_i by n_i u of its own;
//   * from that lower bound the terms that cannot change the sum (below
//     half its quantum) are dropped, each segment packs or keeps its live
//     terms and forms its pairs in the binades its running sum can occupy,
//     exactly as exact_normaliser does within one workgroup, and publishes
//     them with its terms;
//   * a segment whose sum may leave a binade also publishes its runs
//     (seg_runs, for a start anywhere in its bounds).
// Window 0 (of several) walks its own 16 segments from its LDS copy (its
// first one while its other waves form their pairs) and publishes the exact
// sum at its end with the call's tag.  The walker, wave 0 of the job's last
// workgroup, waits for that sum (bounded; if the wait ran out it would walk
// from zero) and sums the other segments in order with the exact running
// sum: runs of segments covered by pairs at once, any other segment by its
// runs (runs_walk).  The sum is exact whatever the estimates.  Then the
// row's candidate path runs again with that S, its LDS partials and
// candidates put back by the walker's other waves during the walk (a row of
// several segments: finalize_rare, path 6).
constexpr uint32_t XS_SPIN = 1u << 16;
constexpr uint32_t XS_RUNW = 256;              // a segment's runs: a lane's (a0, a1, k, 0)
constexpr uint32_t XS_SLOT = TILE + XS_RUNW;   // an LDS copy: terms, then runs
constexpr uint32_t XS_PACKED = 0x80000000u;    // record word 7: packed terms
constexpr uint32_t XS_RUNS = 0x40000000u;      //   runs formed with the terms
constexpr uint32_t XS_CNT = 0x3fffffffu;       //   the terms' count
// The exact running sum from cc over segments s .. se - 1, by one wave (every
// lane returns it): a run of segments whose pair covers the sum's binade and
// keeps it there is added at once, any other segment lane by lane
// (wave_sum_q).  hdr(i, x): word x of segment i's record (0 the header, 1-6
// its pairs, 7 its count and packed bit); T::get4 / T::get16 read a lane's
// terms of a packed / dense segment.
template <class H, class T>
__device__ __forceinline__ float xs_walk(float cc, uint32_t s, uint32_t se, H hdr, T src) {
  const uint32_t lane = threadIdx.x & 63u;
  while (s < se) {
    if (__float_as_uint(cc) >= 0x00800000u) {
      const int eb = binade_of(cc);
      const uint32_t C = (uint32_t)__builtin_ldexpf(cc, 23 - eb);
      const uint32_t js = s + lane;
      Par px = Par{XS_SAT, XS_SAT};
      if (js < se) {
        const uint32_t hj = hdr(js, 0u);
        const int q = eb - ((int)(hj & 0xffffu) - 256);
        if ((hj >> 16) != 0u && q >= 0 && q < (int)(hj >> 16))
          px = Par{hdr(js, 1u + 2u * (uint32_t)q), hdr(js, 2u + 2u * (uint32_t)q)};
      }
      const Par in = wave_par_incl_sat(px);
      const uint32_t inc = (C & 1u) ? in.a1 : in.a0;
      const uint64_t good = __ballot(js < se && C + inc < XS_SAT);
      const uint32_t g = ~good == 0ull ? 64u : (uint32_t)__builtin_ctzll(~good);
      if (g > 0) {
        const uint32_t ig = (uint32_t)__builtin_amdgcn_readlane((int)inc, (int)g - 1);
        cc = __builtin_ldexpf((float)(C + ig), eb - 23);
        s += g;
        continue;
      }
    }
    const uint32_t mts = hdr(s, 7u);
    const uint32_t cnt = mts & XS_CNT;
    // the segment's runs, formed with its terms for the bounds on its start,
    // or formed here from the exact sum
    const bool have = (mts & XS_RUNS) != 0u;
    RunLane r = RunLane{0u, 0u, 0u};
    if (have) r = src.runs(s, lane);
    if (mts & XS_PACKED) {
      float p4[4];
      src.get4(s, lane, p4);
#pragma unroll
      for (uint32_t q = 0; q < 4; ++q) p4[q] = 4 * lane + q < cnt ? p4[q] : 0.0f;
      const uint32_t nl = (cnt + 3u) / 4u;
      if (nl > 0) cc = runs_walk<4>(cc, p4, nl, have ? r : seg_runs<4>(p4, nl, cc, cc));
    } else {
      float p16[16];
      src.get16(s, lane, p16);
      const uint32_t nl = (cnt + 15u) / 16u;
      if (nl > 0) cc = runs_walk<16>(cc, p16, nl, have ? r : seg_runs<16>(p16, nl, cc, cc));
    }
    ++s;
  }
  return cc;
}
// a segment's terms and runs: their LDS copy when it has one, else the
// published ones
struct XsTerms {
  LDS const float* pf;       // [npf][XS_SLOT]: terms, then runs
  LDS const uint32_t* pfs;   // segment -> copy, or EMPTY
  const GLB float* terms;    // [ns][TILE]
  const GLB uint32_t* rw;    // [ns][XS_RUNW]
  __device__ __forceinline__ RunLane runs(uint32_t s, uint32_t lane) const {
    const uint32_t slot = pfs[s];
    const u4v v = slot != EMPTY
                      ? *(LDS const u4v*)((LDS const uint32_t*)pf + (uint64_t)slot * XS_SLOT +
                                          TILE + 4 * lane)
                      : *(const GLB u4v*)(rw + (uint64_t)s * XS_RUNW + 4 * lane);
    return RunLane{v.x, v.y, v.z};
  }
  __device__ __forceinline__ void get4(uint32_t s, uint32_t lane, float (&p)[4]) const {
    const uint32_t slot = pfs[s];
    const f4v v = slot != EMPTY ? *(LDS const f4v*)(pf + (uint64_t)slot * XS_SLOT + 4 * lane)
                                : *(const GLB f4v*)(terms + (uint64_t)s * TILE + 4 * lane);
    p[0] = v.x;
    p[1] = v.y;
    p[2] = v.z;
    p[3] = v.w;
  }
  __device__ __forceinline__ void get16(uint32_t s, uint32_t lane, float (&p)[16]) const {
    const uint32_t slot = pfs[s];
#pragma unroll
    for (uint32_t q = 0; q < 16; q += 4) {
      const f4v v = slot != EMPTY
                        ? *(LDS const f4v*)(pf + (uint64_t)slot * XS_SLOT + 16 * lane + q)
                        : *(const GLB f4v*)(terms + (uint64_t)s * TILE + 16 * lane + q);
      p[q] = v.x;
      p[q + 1] = v.y;
      p[q + 2] = v.z;
      p[q + 3] = v.w;
    }
  }
};
// window 0's own copy of its segments' terms (segment s at s * TILE) and
// runs (at 16 * TILE + s * XS_RUNW)
struct XsOwnTerms {
  LDS const float* t;
  __device__ __forceinline__ RunLane runs(uint32_t s, uint32_t lane) const {
    const u4v v = *(LDS const u4v*)((LDS const uint32_t*)t + 16 * TILE + s * XS_RUNW + 4 * lane);
    return RunLane{v.x, v.y, v.z};
  }
  __device__ __forceinline__ void get4(uint32_t s, uint32_t lane, float (&p)[4]) const {
    const f4v v = *(LDS const f4v*)(t + s * TILE + 4 * lane);
    p[0] = v.x;
    p[1] = v.y;
    p[2] = v.z;
    p[3] = v.w;
  }
  __device__ __forceinline__ void get16(uint32_t s, uint32_t lane, float (&p)[16]) const {
#pragma unroll
    for (uint32_t q = 0; q < 16; q += 4) {
      const f4v v = *(LDS const f4v*)(t + s * TILE + 16 * lane + q);
      p[q] = v.x;
      p[q + 1] = v.y;
      p[q + 2] = v.z;
      p[q + 3] = v.w;
    }
  }
};
template <int DT>
__device__ __forceinline__ void xs_phase() {
  extern __shared__ __align__(16) uint32_t smem[];
  const KCtx kc = kctx_load();
  const Args& a = kc.a;
  const Ws& w = kc.w;
  LDS uint32_t* sm = (LDS uint32_t*)smem;
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wv = (uint32_t)__builtin_amdgcn_readfirstlane((int)(tid >> 6));
  const uint32_t nwin = (a.V + XS_W - 1) / XS_W;
  const uint32_t j = blockIdx.x / nwin, k = blockIdx.x % nwin;
  {
    const GLB uint32_t* rec = G(w.xs_job) + (uint64_t)j * XS_JOB_WORDS;
    if (tid < 17) sm[tid] = rec[tid];
    __syncthreads();
    auto sw = [&](uint32_t i) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)sm[i]); };
    const uint32_t b = sw(0);
    RowP P;
    P.T = __uint_as_float(sw(1));
    P.top_p = __uint_as_float(sw(2));
    P.min_p = __uint_as_float(sw(3));
    P.rp = __uint_as_float(sw(4));
    P.pp = __uint_as_float(sw(5));
    P.fp = __uint_as_float(sw(6));
    P.K = (int32_t)sw(7);
    P.mode = sw(8);
    P.Kc = sw(9);
    const float m = __uint_as_float(sw(10)), L = __uint_as_float(sw(11));
    const float u = __uint_as_float(sw(12));
    const u4v seg_own = u4v{sw(13), sw(14), sw(15), sw(16)};
    __syncthreads();
    const uint32_t maxw = w.xs_maxw;
    GLB float* wsum = G(w.xs_wsum) + (uint64_t)j * maxw;
    GLB uint32_t* wflag = G(w.xs_wflag) + (uint64_t)j * maxw;
    GLB uint32_t* meta = G(w.xs_meta) + (uint64_t)j * maxw * 16 * 8;
    GLB float* terms = G(w.xs_terms) + (uint64_t)j * maxw * 16 * TILE;
    GLB uint32_t* runs = G(w.xs_runs) + (uint64_t)j * maxw * 16 * XS_RUNW;
    const void* row = (const char*)a.logits +
                      (uint64_t)b * a.stride * ((DT & 3) == LLMK_F32 ? 4u : 2u);
    const GLB uint32_t* mrow = a.mask ? G(a.mask) + (uint64_t)b * a.mask_words : nullptr;
    // ---- the window
    // LDS: [0, 64) reductions, 64 flags, [128, 192) the history build's
    // scan, [256, ...) the window's history tables, then the packed terms
    constexpr uint32_t HW = XS_W / 32;
    LDS float* segw = (LDS float*)(sm + 200);   // [NW] all terms
    LDS float* segl = (LDS float*)(sm + 216);   // [NW] live terms
    LDS uint32_t* hb = sm + 256;
    LDS float* comp = (LDS float*)(hb + hist_lds_words(HW)) + XS_CW * wv;
    const uint32_t lo = k * XS_W, hi = umin(lo + XS_W, a.V);
    Hist h;
    hist_carve(h, hb, HW);
    h.lo = lo;
    // the window's logits requested first, the history tables built meanwhile
    const uint32_t e0 = lo + 16 * tid;
    float x[16];
    load16<DT>(row, e0, a.V, x);
    const uint32_t mw = (mrow && e0 < a.V) ? mrow[e0 >> 5] >> (e0 & 16u) : 0xffffffffu;
    if (tid == 0) sm[64] = 0;
    build_history<DT>(a, P, b, row, lo, hi, HW, h, sm + 128, &sm[64]);
    const uint32_t hw = e0 < a.V ? h.bitmap[(e0 - lo) >> 5] >> (e0 & 16u) : 0u;
    float e[16];
    float ls = 0.0f;
#pragma unroll
    for (uint32_t q = 0; q < 16; ++q) {
      float v = x[q];
      if ((hw >> q) & 1u) v = h.pen[h.rank(e0 + q)];
      if (!((mw >> q) & 1u) || !(v > NEG_INF)) v = NEG_INF;
      const float l = (P.T != 1.0f) ? v / P.T : v;
      e[q] = (l == NEG_INF) ? 0.0f : exp_ref<true>(l - m);
      ls += e[q];
    }
    ls = wave_tree_sum(ls);
    if (lane == 0) segw[wv] = ls;
    __syncthreads();
    if (tid == 0) {
      float A = 0.0f;
      for (uint32_t i = 0; i < (uint32_t)NW; ++i) A += segw[i];
      wsum[k] = A;
      __hip_atomic_store(&wflag[k], 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    }
    // ---- the sums before this window (wave 0), then the bounds on c_k
    if (wv == 0) {
      double pre = 0.0;
      uint32_t ok = 1;
      for (uint32_t i0 = 0; i0 < k && ok; i0 += WAVE) {
        const uint32_t i = i0 + lane;
        bool have = i >= k;
        for (uint32_t n = 0; __ballot(!have) != 0ull; ++n) {
          if (n == a.xs_spin) {
            ok = 0;
            break;
          }
          if (!have)
            have = __hip_atomic_load(&wflag[i], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) != 0u;
          if (__ballot(!have) != 0ull) __builtin_amdgcn_s_sleep(2);
        }
        if (!ok) break;
        double v = i < k ? (double)wsum[i] : 0.0;
        v = v + dppd<0x111, 0xf, true>(v);
        v = v + dppd<0x112, 0xf, true>(v);
        v = v + dppd<0x114, 0xf, true>(v);
        v = v + dppd<0x118, 0xf, true>(v);
        v = v + dppd<0x142, 0xa, false>(v);
        v = v + dppd<0x143, 0xc, false>(v);
        pre += readlane_d(v, 63);
      }
      if (lane == 0) {
        sm[66] = ok;
        sm[68] = (uint32_t)__double_as_longlong(pre);
        sm[69] = (uint32_t)((uint64_t)__double_as_longlong(pre) >> 32);
      }
    }
    __syncthreads();
    const double pre = __longlong_as_double((long long)(((uint64_t)sm[69] << 32) | sm[68]));
    double clo = 0.0, chi = 0.0;  // window 0 starts at 0 exactly
    if (k > 0) {
      if (sm[66]) {
        const double d = (double)(lo + XS_W) * 0x1p-24 * 2.02 + 0x1p-30;
        clo = pre * (1.0 - d);
        chi = pre * (1.0 + d);
      } else {
        chi = __builtin_huge_val();  // no estimate: nothing dropped, no pairs
      }
    }
    // ---- the live terms: an e below half the quantum of c_k's lowest
    // possible binade adds nothing (c only grows)
    const float lim = clo >= 0x1p-126 ? (float)__builtin_ldexp(1.0, binade_d(clo) - 24) : 0.0f;
    uint32_t live = 0;
#pragma unroll
    for (uint32_t q = 0; q < 16; ++q)
      if (e[q] > 0.0f && !(e[q] < lim)) live |= 1u << q;
    const uint32_t n = (uint32_t)__popc(live);
    const uint32_t incl = wave_incl_scan(n);
    const uint32_t nw = bcast63u(incl);
    const bool packed = nw <= XS_CW;
    float pk[4];
    if (packed) {
      uint32_t at = incl - n;
#pragma unroll
      for (uint32_t q = 0; q < 16; ++q)
        if ((live >> q) & 1u) comp[at++] = e[q];
      WaveSync::sync();
      const f4v v4 = ((LDS const f4v*)comp)[lane];
      pk[0] = 4 * lane + 0 < nw ? v4.x : 0.0f;
      pk[1] = 4 * lane + 1 < nw ? v4.y : 0.0f;
      pk[2] = 4 * lane + 2 < nw ? v4.z : 0.0f;
      pk[3] = 4 * lane + 3 < nw ? v4.w : 0.0f;
    } else {
#pragma unroll
      for (uint32_t q = 0; q < 16; ++q)
        if (!((live >> q) & 1u)) e[q] = 0.0f;
    }
    const uint32_t sbase = lo + TILE * wv;
    const uint32_t nseg = packed ? nw : (sbase < a.V ? umin(TILE, a.V - sbase) : 0u);
    float ll = 0.0f;
    if (packed) {
      ll = (pk[0] + pk[1]) + (pk[2] + pk[3]);
    } else {
#pragma unroll
      for (uint32_t q = 0; q < 16; ++q) ll += e[q];
    }
    ll = wave_tree_sum(ll);
    if (lane == 0) segl[wv] = ll;
    __syncthreads();
    double blo = clo, bhi = chi;
    for (uint32_t i = 0; i < wv; ++i) {
      blo += (double)segl[i];
      bhi += (double)segl[i];
    }
    const double drift = (double)(TILE * (wv + 1)) * 0x1p-24 * 1.01 + 0x1p-19;
    const double plo = blo * (1.0 - drift), phi = (bhi + (double)segl[wv]) * (1.0 + drift);
    uint32_t hdr = 0;
    Par pr[XS_NB];
#pragma unroll
    for (uint32_t q = 0; q < XS_NB; ++q) pr[q] = Par{0u, 0u};
    if (plo >= 0x1p-126 && phi < 0x1p120) {
      const int elo = binade_d(plo), ehi = binade_d(phi);
      const int nb = ehi - elo + 1;
      if (nb <= (int)XS_NB) {
#pragma unroll
        for (int q = 0; q < (int)XS_NB; ++q) {
          if (q < nb) {
            const Par y = packed ? wave_par_incl_sat(lane_pair<4>(pk, elo + q))
                                 : wave_par_incl_sat(lane_pair<16>(e, elo + q));
            pr[q] = Par{(uint32_t)__builtin_amdgcn_readlane((int)y.a0, 63),
                        (uint32_t)__builtin_amdgcn_readlane((int)y.a1, 63)};
          }
        }
        hdr = (uint32_t)(elo + 256) | ((uint32_t)nb << 16);
      }
    }
    // ---- the runs of a segment the walk may sum lane by lane (no pairs, or
    // pairs in more than one binade), for a start anywhere in [blo, bhi]
    // widened by the drift
    const bool want_runs = (hdr >> 16) != 1u && bhi < 0x1p120 && nseg > 0;
    RunLane rn = RunLane{0u, 0u, 0u};
    if (want_runs) {
      const double slo = blo * (1.0 - drift), shi = bhi * (1.0 + drift);
      rn = packed ? seg_runs<4>(pk, (nseg + 3u) / 4u, slo, shi)
                  : seg_runs<16>(e, (nseg + 15u) / 16u, slo, shi);
    }
    const uint32_t word7 = nseg | (packed ? XS_PACKED : 0u) | (want_runs ? XS_RUNS : 0u);
    // window 0 (of several) starts its own walk here: its first segment's
    // runs were formed for a start at exactly 0, so wave 0 sums them while
    // the other waves form their pairs (sm[73]: the sum, sm[74]: segments
    // done)
    if (k == 0 && wv == 0 && nwin > 1) {
      float c0 = 0.0f;
      if (want_runs)
        c0 = packed ? runs_walk<4>(0.0f, pk, (nseg + 3u) / 4u, rn)
                    : runs_walk<16>(0.0f, e, (nseg + 15u) / 16u, rn);
      if (lane == 0) {
        sm[73] = __float_as_uint(c0);
        sm[74] = want_runs ? 1u : 0u;
      }
    }
    // ---- publish the segment: header, pairs, count, terms, runs
    const uint32_t sg = 16 * k + wv;
    GLB uint32_t* mt = meta + (uint64_t)sg * 8;
    GLB float* tt = terms + (uint64_t)sg * TILE;
    if (lane == 0) {
      mt[0] = hdr;
#pragma unroll
      for (uint32_t q = 0; q < XS_NB; ++q) {
        mt[1 + 2 * q] = pr[q].a0;
        mt[2 + 2 * q] = pr[q].a1;
      }
      mt[7] = word7;
    }
    if (want_runs)
      *(GLB u4v*)(runs + (uint64_t)sg * XS_RUNW + 4 * lane) = u4v{rn.a0, rn.a1, rn.k, 0u};
    if (packed) {
      *(GLB f4v*)(tt + 4 * lane) = f4v{pk[0], pk[1], pk[2], pk[3]};
    } else {
#pragma unroll
      for (uint32_t q = 0; q < 16; q += 4)
        *(GLB f4v*)(tt + 16 * lane + q) = f4v{e[q], e[q + 1], e[q + 2], e[q + 3]};
    }
    // window 0 (of several) keeps its records, terms and runs in LDS too, in
    // the history tables' place (no wave reads them past the barrier before
    // the pairs), for its own walk below
    LDS uint32_t* own = hb;  // [16][8], then [16][TILE] terms, then [16][XS_RUNW] runs
    if (k == 0 && nwin > 1) {
      if (lane == 0) {
        own[8 * wv] = hdr;
#pragma unroll
        for (uint32_t q = 0; q < XS_NB; ++q) {
          own[8 * wv + 1 + 2 * q] = pr[q].a0;
          own[8 * wv + 2 + 2 * q] = pr[q].a1;
        }
        own[8 * wv + 7] = word7;
      }
      if (want_runs)
        *(LDS u4v*)(own + 128 + 16 * TILE + XS_RUNW * wv + 4 * lane) = u4v{rn.a0, rn.a1, rn.k, 0u};
      LDS float* ot = (LDS float*)(own + 128) + TILE * wv;
      if (packed) {
        *(LDS f4v*)(ot + 4 * lane) = f4v{pk[0], pk[1], pk[2], pk[3]};
      } else {
#pragma unroll
        for (uint32_t q = 0; q < 16; q += 4)
          *(LDS f4v*)(ot + 16 * lane + q) = f4v{e[q], e[q + 1], e[q + 2], e[q + 3]};
      }
    }
    // the sum at window 0's end, once window 0 has walked itself: the call's
    // tag (its count of calls + 1) marks it as this call's
    const uint32_t tag = a.epoch + 1u;
    GLB uint32_t* own_sum = G(w.xs_ctl) + XS_PRE + 2 * j;  // (sum, tag)
    // the barrier gathers every wave's stores in this CU's caches; thread 0's
    // arrival then releases them (a write-back of the cache) and, for the
    // last window, acquires the others' (an invalidation the whole
    // workgroup's loads see); one fence per workgroup, not one per wave
    __syncthreads();
    if (tid == 0)
      sm[70] = __hip_atomic_fetch_add(&w.xs_ctl[2 + j], 1u, __ATOMIC_ACQ_REL,
                                      __HIP_MEMORY_SCOPE_AGENT) == nwin - 1
                   ? 1u
                   : 0u;
    __syncthreads();
    if (sm[70]) {
      // ---- the walker: every window's segments, in order
      const uint32_t ns = 16 * nwin;
      LDS uint32_t* segp = sm + 256;         // [ns][8]
      LDS uint32_t* pfs = segp + ns * 8;     // [ns]: LDS copy of a segment's terms, or EMPTY
      LDS uint32_t* pfl = pfs + ns;          // [ns]: the segment of each copy
      LDS float* pf = (LDS float*)(pfl + ns);  // [npf][XS_SLOT]: terms, then runs
      // (below a single-segment row's partials and candidates, which go back
      // in place during the walk)
      const uint32_t lds_top = a.G == 1 ? a.lds_part : a.xs_lds;
      const uint32_t npf = (lds_top - (256 + 10 * ns)) / XS_SLOT;
      // window 0 walks its own segments (below, or first here when it is the
      // last to arrive) and the walk here starts at their end
      const bool from_own = nwin > 1;
      if (k == 0 && from_own) {
        if (wv == 0) {
          const float c = xs_walk(__uint_as_float(sm[73]), sm[74], 16u,
                                  [&](uint32_t i, uint32_t x) { return own[8 * i + x]; },
                                  XsOwnTerms{(LDS const float*)(own + 128)});
          if (lane == 0) sm[75] = __float_as_uint(c);
        }
        __syncthreads();
      }
      // the segments' headers, and the terms of window 0's segments when the
      // walk starts at zero (from there window 0 crosses a binade at each
      // doubling, so the walk sums most of its segments lane by lane), in
      // one round of loads
      const uint32_t n0 = from_own ? 0u : umin(16u, npf);
      {
        uint32_t mv[8];
        float tv[16];
        uint32_t rv[4];
#pragma unroll
        for (uint32_t q = 0; q < 8; ++q) {
          const uint32_t i = tid + q * NT;
          mv[q] = i < ns * 8 ? meta[i] : 0u;
        }
#pragma unroll
        for (uint32_t q = 0; q < 16; ++q) tv[q] = q < n0 ? terms[q * TILE + tid] : 0.0f;
#pragma unroll
        for (uint32_t q = 0; q < 4; ++q) rv[q] = 4 * q < n0 ? runs[q * NT + tid] : 0u;
#pragma unroll
        for (uint32_t q = 0; q < 8; ++q) {
          const uint32_t i = tid + q * NT;
          if (i < ns * 8) segp[i] = mv[q];
        }
#pragma unroll
        for (uint32_t q = 0; q < 16; ++q)
          if (q < n0) pf[q * XS_SLOT + tid] = tv[q];
        // runs of segments 4q .. 4q + 3: thread t holds word t of them
#pragma unroll
        for (uint32_t q = 0; q < 4; ++q) {
          const uint32_t sq = 4 * q + tid / XS_RUNW;
          if (sq < n0) ((LDS uint32_t*)pf)[sq * XS_SLOT + TILE + tid % XS_RUNW] = rv[q];
        }
      }
      __syncthreads();
      // then the other segments past window 0 that the walk may sum lane by
      // lane (no pairs, or pairs in more than one binade), as many as fit (the
      // rest are read when the walk reaches them)
      const uint32_t sfirst = from_own ? 16u : n0;
      if (wv == 0) {
        uint32_t used = n0;
        for (uint32_t s0 = 0; s0 < ns; s0 += WAVE) {
          const uint32_t si = s0 + lane;
          const bool want = si >= sfirst && si < ns && (segp[8 * si] >> 16) != 1u;
          const uint32_t r = used + (uint32_t)__popcll(__ballot(want) & ((1ull << lane) - 1ull));
          if (si < n0) pfs[si] = si;
          else if (si < ns) pfs[si] = (want && r < npf) ? r : EMPTY;
          if (want && r < npf) pfl[r] = si;
          used += (uint32_t)__popcll(__ballot(want));
        }
        if (lane == 0) sm[72] = umin(used, npf);
      }
      __syncthreads();
      const uint32_t nused = sm[72];
      // eight segments' loads in flight before their stores (thread t copies
      // element t of each; past a segment's count the copy is never read)
      for (uint32_t s0 = n0; s0 < nused; s0 += 8) {
        float v[8];
        uint32_t rv[2];
#pragma unroll
        for (uint32_t q = 0; q < 8; ++q)
          v[q] = s0 + q < nused ? terms[(uint64_t)pfl[s0 + q] * TILE + tid] : 0.0f;
#pragma unroll
        for (uint32_t q = 0; q < 2; ++q) {
          const uint32_t sq = s0 + 4 * q + tid / XS_RUNW;
          rv[q] = sq < nused ? runs[(uint64_t)pfl[sq] * XS_RUNW + tid % XS_RUNW] : 0u;
        }
#pragma unroll
        for (uint32_t q = 0; q < 8; ++q)
          if (s0 + q < nused) pf[(s0 + q) * XS_SLOT + tid] = v[q];
#pragma unroll
        for (uint32_t q = 0; q < 2; ++q) {
          const uint32_t sq = s0 + 4 * q + tid / XS_RUNW;
          if (sq < nused) ((LDS uint32_t*)pf)[sq * XS_SLOT + TILE + tid % XS_RUNW] = rv[q];
        }
      }
      __syncthreads();
      // a single-segment row's LDS partials and candidates back in place
      // (waves 1-15, while wave 0 walks)
      if (a.G == 1 && wv != 0) {
        const GLB uint32_t* sv = G(w.xs_save) + (uint64_t)j * XS_SAVE;
        for (uint32_t i = tid - WAVE; i < XS_SAVE; i += NT - WAVE) sm[a.lds_part + i] = sv[i];
      }
      if (wv == 0) {
        // window 0's sum at its end (a bounded wait; if it runs out, the
        // walk starts at zero and reads window 0's terms from memory)
        float c0 = 0.0f;
        uint32_t s0 = 0;
        if (k == 0 && from_own) {
          c0 = __uint_as_float(sm[75]);
          s0 = 16;
        } else if (from_own) {
          for (uint32_t n = 0; n < a.xs_spin; ++n) {
            const uint32_t t = __hip_atomic_load(own_sum + 1, __ATOMIC_ACQUIRE,
                                                 __HIP_MEMORY_SCOPE_AGENT);
            if ((uint32_t)__builtin_amdgcn_readfirstlane((int)t) == tag) {
              c0 = __uint_as_float(
                  (uint32_t)__builtin_amdgcn_readfirstlane((int)own_sum[0]));
              s0 = 16;
              break;
            }
            __builtin_amdgcn_s_sleep(2);
          }
        }
        const float cc = xs_walk(c0, s0, ns,
                                 [&](uint32_t i, uint32_t x) { return segp[8 * i + x]; },
                                 XsTerms{pf, pfs, terms, runs});
        if (lane == 0) sm[71] = __float_as_uint(cc);
      }
      __syncthreads();
      const float S = __uint_as_float(sm[71]);
      // the job's counters back to zero for the next call
      if (tid == 0) __hip_atomic_store(&w.xs_ctl[2 + j], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      for (uint32_t i = tid; i < nwin; i += NT) wflag[i] = 0u;
      __syncthreads();
      // the row's candidate path: for a single-segment row here (its history
      // never outgrew its tables; its partials and candidates are back), the
      // rest through finalize_rare (a call: its register saves cost
      // microseconds)
      if (a.G == 1) {
        const uint32_t path = candidate_paths<DT>(a, w, b, P, S, m, L, u, seg_own, false, sm);
        if (path != 0) finalize_rare<DT>(b, P, S, m, L, u, seg_own, false, path);
      } else {
        finalize_rare<DT>(b, P, S, m, L, u, seg_own, false, 6u);
      }
    } else if (k == 0 && wv == 0) {
      // ---- window 0's own walk over its LDS copy, on from its first segment
      const float cc = xs_walk(__uint_as_float(sm[73]), sm[74], 16u,
                               [&](uint32_t i, uint32_t x) { return own[8 * i + x]; },
                               XsOwnTerms{(LDS const float*)(own + 128)});
      if (lane == 0) {
        own_sum[0] = __float_as_uint(cc);
        __hip_atomic_store(own_sum + 1, tag, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

// seg_own: for a single-segment row, this workgroup's (count, beta, flags);
// u: the row's uniform (loaded with the parameters, so that no global load
// is outstanding at the finalize's barriers).
//
// The normaliser S: 1 on a row that top-k renormalises (0 < top_k < V,
// sampler.rs:80-89: every probability is divided by the top-k sum before
// any step reads it, so S cancels in exact arithmetic) until its band check
// fails, then the reference's own; 0 for a row whose logits are
// all -inf; else the reference's own sequential f32 sum in index order
// (exact_normaliser; sampler.rs:66).  A single-segment row still holds the
// whole row's history tables from its stream phase; a row of several
// segments rebuilds them first.
template <int DT>
__device__ __forceinline__ void finalize_row(const Args& a, const Ws& w, uint32_t b,
                                             const RowP& P, bool have_vt, u4v seg_own, float u,
                                             LDS uint32_t* smem) {
  const uint32_t tid = threadIdx.x;
  const int lane = (int)(tid & 63), wv = (int)(tid >> 6);
  const FinLds f = fin_carve(smem);
  const uint32_t nslots = a.ntiles + (have_vt ? a.nchunks : 0u);
  // ---- wave 0: the row maximum L (and the greedy token, unless a segment's
  // history outgrew its tables: the slow path then materialises the row)
  if (wv == 0) {
    const GLB f2v* part = G(w.tile_part) + (uint64_t)b * MAX_SLOTS;
    LDS const f2v* lpart = (LDS const f2v*)(smem + a.lds_part);
    float L = NEG_INF;
    uint32_t hov = 0;
    if (P.mode == MODE_GREEDY) {
      uint32_t flg = 0;
      if (a.G == 1) flg = seg_own.z;
      else if ((uint32_t)lane < a.G) flg = G(w.seg_meta)[row_seg_to_wg(a, b, (uint32_t)lane)].z;
      hov = __ballot((flg & FLAG_HIST_OVERFLOW) != 0) != 0ull ? 1u : 0u;
    }
    if (hov) {
    } else if (P.mode == MODE_GREEDY) {
      for (uint32_t c = (uint32_t)lane; c < nslots; c += WAVE) {
        const f2v q = a.G == 1 ? lpart[c] : part[c];
        f.tl[c] = q.x;
        f.ts[c] = q.y;
        L = fmaxf(L, q.x);
      }
      L = wave_max(L);
      WaveSync::sync();
      // sampler.rs:40-50: the first index holding the maximum
      uint32_t bi = EMPTY;
      for (uint32_t c = (uint32_t)lane; c < nslots; c += WAVE)
        if (f.tl[c] == L) bi = umin(bi, __float_as_uint(f.ts[c]));
      bi = wave_min_u32(bi);
      if (bi == EMPTY) bi = 0;
      if (lane == 0) {
        G(a.out_tok)[b] = bi;
        if (a.out_cnt) G(a.out_cnt)[b] = 1;
        if (a.out_cap) {
          if (a.out_ids) G(a.out_ids)[(uint64_t)b * a.out_cap] = bi;
          if (a.out_probs) G(a.out_probs)[(uint64_t)b * a.out_cap] = 1.0f;
        }
      }
    } else {
      for (uint32_t c = (uint32_t)lane; c < nslots; c += WAVE)
        L = fmaxf(L, a.G == 1 ? lpart[c].x : part[c].x);
      L = wave_max(L);
    }
    if (lane == 0) {
      g_bcast[0] = __float_as_uint(L);
      g_bcast[1] = hov;
    }
  }
  __syncthreads();
  if (P.mode == MODE_GREEDY && g_bcast[1] == 0) return;
  const float L = __uint_as_float(g_bcast[0]);
  const float m = (P.T != 1.0f) ? L / P.T : L;
  const bool topk = P.K > 0 && (uint32_t)P.K < a.V;
  float S = 1.0f;
  bool rebuilt_ovf = false;
  if (L == NEG_INF) {
    S = 0.0f;
  } else if (!topk) {
    Hist h;
    bool have_hist = have_vt;
    LDS uint32_t* sc = smem;  // below the tables in both layouts
    if (a.G == 1) {
      // the stream phase's tables: the stream layout's history words
      hist_carve(h, smem + 64 + M_NMISC + NBINS + 64, a.ntiles * 32);
      h.lo = 0;
    } else {
      LDS uint32_t* hb = smem + 128 + 256 + NW * 256 + SLOW_BINS;  // the slow path's layout
      const uint32_t nwords = (a.V + 31) / 32;
      hist_carve(h, hb, nwords);
      h.lo = 0;
      if (tid == 0) sc[64] = 0;
      const void* row = (const char*)a.logits +
                        (uint64_t)b * a.stride * ((DT & 3) == LLMK_F32 ? 4u : 2u);
      build_history<DT>(a, P, b, row, 0, a.V, nwords, h, sc + 128, &sc[64]);
      have_hist = true;  // built (empty when the row has no penalised history)
      // the whole row's history outgrows the tables (the segments' did not)
      rebuilt_ovf = (sc[64] & FLAG_HIST_OVERFLOW) != 0;
    }
    const void* row = (const char*)a.logits +
                      (uint64_t)b * a.stride * ((DT & 3) == LLMK_F32 ? 4u : 2u);
    if (!rebuilt_ovf)
      S = exact_normaliser<DT>(row, a.mask ? a.mask + (uint64_t)b * a.mask_words : nullptr,
                               a.V, P.T, m, h.bitmap, h.pre, h.pen, have_hist, sc);
  }
  // S = 1 stands in for the reference's S on a row that top-k renormalises
  const bool approx = topk && L != NEG_INF;
  const uint32_t path =
      candidate_paths<DT>(a, w, b, P, S, m, L, u, seg_own, approx, smem, rebuilt_ovf);
  if (path == 0) return;
  // the slow path, (4) the band check could not prove S = 1: the reference's
  // S, then the candidate path again, or (5) the row's history outgrew the
  // tables: the slow path materialises the row
  kctx_fill();
  __syncthreads();
  finalize_rare<DT>(b, P, S, m, L, u, seg_own, approx, path);
}

// ---------------------------------------------------------------------------
// Per-tile reduction of the vocabulary tiles
// ---------------------------------------------------------------------------
struct TileEnv {
  RowP P;
  uint32_t V;
  bool collect;
  uint32_t recompute_at;
  LDS uint32_t* misc;
  LDS uint32_t* hf;
  LDS uint32_t* hcoarse;
  GLB u2v* cbuf;
  GLB f2v* part;
  LDS f2v* lpart;  // non-null for a single-segment row: partials kept in LDS
  LDS u2v* lcand;  //   and its first LCAP candidates
};
__device__ __forceinline__ void put_part(const TileEnv& E, uint32_t slot, f2v x) {
  if (E.lpart) E.lpart[slot] = x;
  else E.part[slot] = x;
}
__device__ __forceinline__ void put_cand(const TileEnv& E, uint32_t pos, u2v x) {
  if (E.lcand && pos < LCAP) E.lcand[pos] = x;
  else E.cbuf[pos] = x;
}

// v[j], j = 4r + q: the lane's values at tile positions 256r + 4*lane + q,
// excluded positions already -inf.  idx(j): the vocabulary index of value j
// (EMPTY or >= V for a position that holds no token).  Writes the slot's
// partial (tile max, tree sum of 2^((v - max) c2)) -- or (max, first index of
// the max) for greedy rows -- and appends candidates above the row's rising
// threshold.  `since` is the wave's count of appends since its last threshold
// update (EMPTY before its first counted tile).
//
// nr (wave-uniform, 1..4): runs r >= nr hold only -inf positions; each of
// their terms is exactly exp2_f(-inf) = 2^-125, so such a run sums to 2^-123
// and is not evaluated.
template <class IDX>
__device__ __forceinline__ void tile_reduce(const TileEnv& E, const float (&v)[16],
                                            uint32_t slot, const IDX& idx,
                                            uint32_t& since, int lane, uint32_t nr = 4) {
  float lm = NEG_INF;
  if (E.P.mode == MODE_SAMPLE) {
    // v_maximum3_f32 propagates NaN at the cost of v_max3_f32, so one
    // compare per lane finds a logit that makes the reference's
    // probabilities NaN: NaN, or +inf (whose l - max is inf - inf).
    // Masked logits are -inf by now.  Greedy rows return before the
    // reference's NaN check (sampler.rs:40-50, :74-76).
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if ((uint32_t)(j >> 2) < nr) lm = __builtin_elementwise_maximum(lm, v[j]);
    if (__ballot(!(lm < __builtin_huge_valf()))) {
      if (lane == 0) __atomic_fetch_or(&E.misc[M_FLAGS], FLAG_NAN, __ATOMIC_RELAXED);
      lm = NEG_INF;  // the tile's maximum with NaN read as -inf
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if ((uint32_t)(j >> 2) < nr) lm = fmaxf(lm, v[j]);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if ((uint32_t)(j >> 2) < nr) lm = fmaxf(lm, v[j]);
  }
  lm = wave_max(lm);
  if (E.P.mode == MODE_GREEDY) {
    uint32_t bi = EMPTY;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const bool hit = (v[j] == lm) || (lm == NEG_INF && !(v[j] > NEG_INF));
      if (hit) {
        const uint32_t e = idx(j);
        if (e < E.V) bi = umin(bi, e);
      }
    }
    bi = wave_min_u32(bi);
    if (lane == 0) put_part(E, slot, f2v{lm, __uint_as_float(bi)});
    return;
  }
  if (lane == 0) put_part(E, slot, f2v{lm, 0.0f});
  if (!E.collect) return;
  // ---- candidates above the rising histogram threshold
  uint32_t beta = __atomic_load_n(&E.misc[M_BETA], __ATOMIC_RELAXED);
  float th = theta_of(beta);
  if (!(lm >= th)) return;  // no element of this tile can pass
  bool counted = false;
  if (since == EMPTY) {
    // a wave's first such tile: count each lane's maximum (a subset of the
    // row, so the counts stay lower bounds), raise the threshold, then
    // append without counting again
    float lmax = NEG_INF;
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if ((uint32_t)(j >> 2) < nr) lmax = fmaxf(lmax, v[j]);
    if (lmax >= th) {
      const uint32_t bin = fkey(lmax) >> BIN_SHIFT;
      __atomic_fetch_add(&E.hf[bin], 1u, __ATOMIC_RELAXED);
      __atomic_fetch_add(&E.hcoarse[bin >> (CBIN_SHIFT - BIN_SHIFT)], 1u, __ATOMIC_RELAXED);
    }
    const uint32_t nbeta = compute_beta(E.hcoarse, E.hf, E.P.Kc, lane);
    if (nbeta > beta) {
      if (lane == 0) __atomic_fetch_max(&E.misc[M_BETA], nbeta, __ATOMIC_RELAXED);
      beta = nbeta;
      th = theta_of(beta);
    }
    since = 0;
    counted = true;
  }
  uint64_t mk[16];
  uint32_t npass = 0;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    mk[j] = ((uint32_t)(j >> 2) < nr) ? __ballot(v[j] >= th) : 0ull;
    npass += (uint32_t)__popcll(mk[j]);
  }
  if (npass == 0) return;
  uint32_t base = 0;
  if (lane == 0) base = __atomic_fetch_add(&E.misc[M_CCOUNT], npass, __ATOMIC_RELAXED);
  base = (uint32_t)__builtin_amdgcn_readfirstlane((int)base);
  if (base + npass > CAND_CAP) {
    if (lane == 0) __atomic_fetch_or(&E.misc[M_FLAGS], FLAG_OVERFLOW, __ATOMIC_RELAXED);
    return;
  }
  // append, and count what was appended in the histogram
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    if (mk[j]) {
      if (v[j] >= th) {
        if (!counted) {
          const uint32_t bin = fkey(v[j]) >> BIN_SHIFT;
          __atomic_fetch_add(&E.hf[bin], 1u, __ATOMIC_RELAXED);
          __atomic_fetch_add(&E.hcoarse[bin >> (CBIN_SHIFT - BIN_SHIFT)], 1u, __ATOMIC_RELAXED);
        }
        put_cand(E, base + lanes_below(mk[j]), u2v{__float_as_uint(v[j]), idx(j)});
      }
      base += (uint32_t)__popcll(mk[j]);
    }
  }
  if (counted) return;
  since += npass;
  if (since >= E.recompute_at) {
    since = 0;
    const uint32_t nbeta = compute_beta(E.hcoarse, E.hf, E.P.Kc, lane);
    if (nbeta > beta && lane == 0) __atomic_fetch_max(&E.misc[M_BETA], nbeta, __ATOMIC_RELAXED);
  }
}

// Sets v to -inf where bit (sh + q) of x is set (x: one exclusion word).
__device__ __forceinline__ float exclude(float v, uint32_t x, uint32_t pos) {
  const uint32_t m = (uint32_t)__builtin_amdgcn_sbfe((int)x, pos, 1);
  uint32_t r;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(m), "v"(0xff800000u), "v"(__float_as_uint(v)));
  return __uint_as_float(r);
}

// ---------------------------------------------------------------------------
// Virtual tiles: the history tokens of one 16-tile chunk, reduced by one
// wave.  The chunk's j-th token (in increasing id) belongs to lane j mod 64,
// which sums its terms sequentially in that order; the lanes are combined by
// a balanced tree.
// ---------------------------------------------------------------------------
constexpr int VB = 8;  // gathers in flight per thread

// The penalised, masked logit of every history rank r < U into pen[r] (over
// the counts), by the first nw waves of the workgroup: VB gathers in flight
// per thread, then the arithmetic.
template <int DT>
__device__ __forceinline__ void gather_penalised(const Args& a, const RowP& P, uint32_t b,
                                                 const void* row, uint32_t U, const Hist& h,
                                                 bool need_cnt, uint32_t nw,
                                                 LDS uint32_t* flags) {
  const uint32_t tid = threadIdx.x, step = nw * WAVE;
  const GLB uint32_t* mrow = a.mask ? G(a.mask) + (uint64_t)b * a.mask_words : nullptr;
  LDS const uint32_t* cnt = (LDS const uint32_t*)h.pen;
  for (uint32_t r0 = 0; r0 < U; r0 += VB * step) {
    const uint32_t nr = (U - r0 + step - 1) / step;  // rounds holding ranks (uniform)
    uint32_t tk[VB], mw[VB];
    float x[VB];
#pragma unroll
    for (int i = 0; i < VB; ++i) {
      const uint32_t r = r0 + i * step + tid;
      tk[i] = ((uint32_t)i < nr && r < U) ? h.tokr[r] : EMPTY;
    }
#pragma unroll
    for (int i = 0; i < VB; ++i) {
      x[i] = 0.0f;
      mw[i] = 0xffffffffu;
      if ((uint32_t)i < nr) {
        x[i] = tk[i] != EMPTY ? load_logit<DT>(row, tk[i]) : 0.0f;
        if (tk[i] != EMPTY && mrow) mw[i] = mrow[tk[i] >> 5];
      }
    }
#pragma unroll
    for (int i = 0; i < VB; ++i) {
      const uint32_t r = r0 + i * step + tid;
      if ((uint32_t)i < nr && tk[i] != EMPTY) {
        const bool allowed = (mw[i] >> (tk[i] & 31)) & 1u;
        if (allowed && !(x[i] < __builtin_huge_valf()) && P.mode == MODE_SAMPLE)
          __atomic_fetch_or(flags, FLAG_NAN, __ATOMIC_RELAXED);
        float y = (x[i] > NEG_INF) ? x[i] : NEG_INF;  // NaN acts as -inf
        y = penalize(y, P, need_cnt ? cnt[r] : 1u);
        if (!allowed) y = NEG_INF;
        h.pen[r] = y;
      }
    }
  }
}

// The virtual tile of chunk kk of the segment: its history tokens are the
// ranks [r0, r1) (pre at the chunk's first word and past its last), their
// penalised values already in pen[]; lane L takes ranks r0 + L, r0 + L + 64,
// ... in increasing order.  The maximum, then the terms summed per lane in
// rank order and as a balanced tree over the lanes, then the candidates.
__device__ __forceinline__ void vtile_chunk(const Args& a, uint32_t t0, uint32_t nwords,
                                         uint32_t kk, uint32_t U, const Hist& h,
                                         const TileEnv& E, int lane) {
  const uint32_t wf = 512u * kk;
  const uint32_t r0 = h.pre[wf];
  const uint32_t r1 = wf + 512u < nwords ? (uint32_t)h.pre[wf + 512u] : U;
  const uint32_t n = r1 - r0;
  const uint32_t slot = a.ntiles + t0 / CHUNK_TILES + kk;
  const bool greedy = E.P.mode == MODE_GREEDY;
  LDS const float* pen = h.pen + r0;
  LDS const uint32_t* tokr = h.tokr + r0;
  float lm = NEG_INF;
  for (uint32_t r = (uint32_t)lane; r < n; r += 64u) lm = fmaxf(lm, pen[r]);
  lm = wave_max(lm);
  if (greedy) {
    // the first (lowest) token holding the maximum; all -inf: the first token
    uint32_t bi = EMPTY;
    for (uint32_t r = (uint32_t)lane; r < n; r += 64u) {
      const float y = pen[r];
      if (y == lm || (lm == NEG_INF && !(y > NEG_INF))) bi = umin(bi, tokr[r]);
    }
    bi = wave_min_u32(bi);
    if (lane == 0) put_part(E, slot, f2v{lm, __uint_as_float(bi)});
    return;
  }
  if (lane == 0) put_part(E, slot, f2v{lm, 0.0f});
  if (!E.collect || lm == NEG_INF) return;
  // ---- candidates: the chunk's history tokens at or above the threshold
  const float th = theta_of(__atomic_load_n(&E.misc[M_BETA], __ATOMIC_RELAXED));
  if (!(lm >= th)) return;
  for (uint32_t j0 = 0; j0 < n; j0 += 64u) {
    const uint32_t r = j0 + (uint32_t)lane;
    const float y = r < n ? pen[r] : NEG_INF;
    const bool keep = r < n && y >= th;
    const uint64_t mk = __ballot(keep);
    if (!mk) continue;
    const uint32_t tot = (uint32_t)__popcll(mk);
    uint32_t base = 0;
    if (lane == 0) base = __atomic_fetch_add(&E.misc[M_CCOUNT], tot, __ATOMIC_RELAXED);
    base = (uint32_t)__builtin_amdgcn_readfirstlane((int)base);
    if (base + tot > CAND_CAP) {
      if (lane == 0) __atomic_fetch_or(&E.misc[M_FLAGS], FLAG_OVERFLOW, __ATOMIC_RELAXED);
      return;
    }
    if (keep) {
      const uint32_t bin = fkey(y) >> BIN_SHIFT;
      __atomic_fetch_add(&E.hf[bin], 1u, __ATOMIC_RELAXED);
      __atomic_fetch_add(&E.hcoarse[bin >> (CBIN_SHIFT - BIN_SHIFT)], 1u, __ATOMIC_RELAXED);
      put_cand(E, base + lanes_below(mk), u2v{__float_as_uint(y), tokr[r]});
    }
  }
}

// ---------------------------------------------------------------------------
// The kernels
// ---------------------------------------------------------------------------
// Phase 1, the launch after the sampling launch: the S of the rows whose
// band check failed.  Most calls have none; a workgroup without a job ends
// before any call (a call saves the callee's registers).
template <int DT>
__global__ __launch_bounds__(NT) void xs_kernel(Args a, Ws w) {
  const uint32_t nwin = (a.V + XS_W - 1) / XS_W;
  if (threadIdx.x == 0)
    g_bcast[2] = __hip_atomic_load(&w.xs_ctl[a.epoch & 1u], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (blockIdx.x / nwin < umin(g_bcast[2], a.xs_cap)) {
    exp_tab_init();
    softcap_init<DT>(a);
    kctx_fill();
    __syncthreads();
    xs_phase<DT>();
  }
}

template <int DT>
__global__ __launch_bounds__(NT) void stream_kernel(Args a, Ws w) {
  extern __shared__ __align__(16) uint32_t smem[];
  // the next call's job count starts at zero (nothing reads it in this call)
  if (blockIdx.x == 0 && threadIdx.x == 0)
    __hip_atomic_store(&w.xs_ctl[(a.epoch + 1u) & 1u], 0u, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  const uint32_t tid = threadIdx.x;
  const int lane = (int)(tid & 63);
  const int wv = __builtin_amdgcn_readfirstlane((int)(tid >> 6));  // wave-uniform
  uint32_t b, g;
  wg_to_row_seg(a, blockIdx.x, b, g);
  // The row's parameters and history extent, ahead of every tile request
  // (behind them they would take microseconds).
  const RowIn rin = load_row(a, b);
  const RowP P = row_params(a, rin);
  const float u_row = rin.u;
  const uint32_t h0 = rin.h0;
  uint32_t h1 = a.hlen ? h0 + rin.hl : rin.hn;
  const uint32_t t0 = g * a.tps;
  const uint32_t t1 = min(t0 + a.tps, a.ntiles);
  const uint32_t lo = t0 * TILE, hi = min(a.V, t1 * TILE);
  LDS uint32_t* sm = (LDS uint32_t*)smem;
  LDS uint32_t* red = sm;                    // 64
  LDS uint32_t* misc = red + 64;             // M_NMISC
  LDS uint32_t* hf = misc + M_NMISC;         // NBINS
  LDS uint32_t* hcoarse = hf + NBINS;        // 64
  LDS uint32_t* hb = hcoarse + 64;           // history tables
  const uint32_t nwords = (t1 - t0) * 32;
  Hist h;
  hist_carve(h, hb, nwords);
  LDS uint32_t* btot = hb + hist_lds_words(nwords);  // NW words
  h.lo = lo;
  // Waves 0..TW-1 load the history tokens (TQ per lane per pass); every
  // wave then requests its first tile.
  constexpr uint32_t TW = 8;
  constexpr int TQ = 4;  // tokens per lane per pass
  const void* row = (const char*)a.logits +
                    (uint64_t)b * a.stride * ((DT & 3) == LLMK_F32 ? 4u : 2u);
  const uint32_t* mrow = a.mask ? a.mask + (uint64_t)b * a.mask_words : nullptr;
  // One tile in flight per wave: 16 waves per CU already keep HBM busy, and
  // a deeper queue only adds latency to every other load (the history
  // tokens and their logits, instruction fetches) and to the last tiles
  // (measured: C3 40.1 -> 38.7 us, C5 165 -> 159 us against two per wave).
  Raw ra;
  uint32_t ta = t0 + (uint32_t)wv;
  ta = ta < t1 ? ta : EMPTY;
  const bool tok_wave = (uint32_t)wv < TW;
  if (P.mode == MODE_INVALID) {
    if (g == 0 && tid == 0) {
      a.out_tok[b] = LLMK_INVALID_TOKEN;
      if (a.out_cnt) a.out_cnt[b] = 0;
      atomicOr(w.status, LLMK_STATUS_INVALID_PARAMS);
    }
    return;
  }
  const bool need_pen = P.rp != 1.0f || P.pp != 0.0f || P.fp != 0.0f;
  if (!need_pen) h1 = h0;
  // history tokens exist: their positions are excluded from the vocabulary
  // tiles and reduced in virtual tiles, one per 16-tile chunk
  const bool have = h1 > h0;
  const bool need_cnt = have && P.fp != 0.0f;
  // no more distinct history tokens than ranks: no token can be dropped
  const bool early = h1 - h0 <= U_MAX;
  const bool collect = P.mode == MODE_SAMPLE && P.Kc > 0;
  TileEnv E;
  E.P = P;
  E.V = a.V;
  E.collect = collect;
  E.recompute_at = P.Kc / 4 > 8 ? P.Kc / 4 : 8;
  E.misc = misc;
  E.hf = hf;
  E.hcoarse = hcoarse;
  E.cbuf = G(w.cand) + (uint64_t)blockIdx.x * CAND_CAP;
  E.part = G(w.tile_part) + (uint64_t)b * MAX_SLOTS;
  E.lpart = a.G == 1 ? (LDS f2v*)(smem + a.lds_part) : nullptr;
  E.lcand = a.G == 1 ? (LDS u2v*)(smem + a.lds_cand) : nullptr;
  const uint32_t nch = (nwords + 511) / 512;  // chunks of this segment
  uint32_t tk[TQ], hc[TQ];
#pragma unroll
  for (int q = 0; q < TQ; ++q) {
    tk[q] = EMPTY;
    hc[q] = 1u;
  }
  if (tok_wave && have) {
#pragma unroll
    for (int q = 0; q < TQ; ++q) {
      const uint32_t i = h0 + q * (TW * WAVE) + tid;
      tk[q] = i < h1 ? G(a.htok)[i] : EMPTY;
      if (need_cnt && a.hcnt) hc[q] = i < h1 ? G(a.hcnt)[i] : 1u;
    }
  }
  if (collect) {
    for (uint32_t i = tid; i < NBINS; i += NT) hf[i] = 0;
    if (tid < 64) hcoarse[tid] = 0;
  }
  if (tid < M_NMISC) misc[tid] = 0;
  exp_tab_init();
  softcap_init<DT>(a);
  if (have) {
    for (uint32_t i = tid; i < nwords; i += NT) h.bitmap[i] = 0;
    if (need_cnt)
      for (uint32_t i = tid; i < U_MAX; i += NT) ((LDS uint32_t*)h.pen)[i] = 0;
  }
  // The history tokens arrive before any tile is requested: behind the first
  // tiles of every workgroup they would take several microseconds, and no
  // tile can be reduced before the tables are built.
  if (tok_wave) {
#pragma unroll
    for (int q = 0; q < TQ; ++q) asm volatile("" ::"v"(tk[q]));
  }
  __syncthreads();
  float pf[TQ];
  uint32_t pm[TQ];
#pragma unroll
  for (int q = 0; q < TQ; ++q) {
    pf[q] = 0.0f;
    pm[q] = 0xffffffffu;
  }
  // Without history, the tiles now.  With history, they are requested after
  // the bitmap barrier: requests queued ahead of the history tokens and
  // their logits would delay them by microseconds, and the tables cannot be
  // built without them.
  if (!have) {
    if (ta != EMPTY) load_tile<DT>(a, row, mrow, h, ta, lane, ra);
  }
  // The history tables: the bitmap of the segment's history tokens, their
  // ranks, for the frequency penalty occurrence counts by rank, and the
  // penalised logits by rank; then the virtual tiles (one per 16-tile chunk).
  if (have) {
    const uint32_t step = TQ * TW * WAVE;
    // fn(token, history index)
    auto each_token = [&](auto&& fn) __attribute__((always_inline)) {
      // the first pass from registers (no load in flight but the tiles'),
      // the rest loaded here
#pragma unroll
      for (int q = 0; q < TQ; ++q)
        if (tk[q] >= lo && tk[q] < hi) fn(tk[q], h0 + q * (TW * WAVE) + tid);
      for (uint32_t c0 = h0 + step; c0 < h1; c0 += step) {
#pragma unroll
        for (int q = 0; q < TQ; ++q) {
          const uint32_t i = c0 + q * (TW * WAVE) + tid;
          const uint32_t t = (i < h1) ? G(a.htok)[i] : EMPTY;
          if (t >= lo && t < hi) fn(t, i);
        }
      }
    };
    // Every history token held in tk[] (one pass): the token waves keep
    // their tokens' logits in registers and place them by rank themselves.
    const bool one_pass = early && h1 - h0 <= step;
    if (tok_wave) {
      each_token([&](uint32_t t, uint32_t) {
        __atomic_fetch_or(&h.bitmap[(t - lo) >> 5], 1u << (t & 31), __ATOMIC_RELAXED);
      });
      // the logits (and allow-mask words) of the first pass's history
      // tokens, requested now, ahead of every tile (after the insertions,
      // which must not wait for them); token waves only: a wait that the
      // others executed, even with no lane loading, would wait for their
      // tiles
#pragma unroll
      for (int q = 0; q < TQ; ++q)
        if (tk[q] >= lo && tk[q] < hi) {
          pf[q] = load_logit<DT>(row, tk[q]);
          if (one_pass && mrow) pm[q] = G(mrow)[tk[q] >> 5];
        }
    }
    __syncthreads();
    // the token waves of the early multi-pass path request theirs after the
    // tables; in one pass the loads of the tokens' logits come first in
    // every token wave, so waiting for them does not wait for its tiles
    if (!(early && tok_wave) || one_pass) {
      if (ta != EMPTY) load_tile<DT>(a, row, mrow, h, ta, lane, ra);
    }
    auto counts = [&]() __attribute__((always_inline)) {
      each_token([&](uint32_t t, uint32_t i) {
        const uint32_t o = t - lo, wd = h.bitmap[o >> 5], bit = 1u << (o & 31);
        if (wd & bit) {  // not dropped by the rank limit
          const uint32_t r = h.pre[o >> 5] + (uint32_t)__popc(wd & (bit - 1u));
          __atomic_fetch_add(&((LDS uint32_t*)h.pen)[r], hist_weight(a, i), __ATOMIC_RELAXED);
        }
      });
    };
    if (early) {
      // At most U_MAX distinct tokens: the bitmap is final, so the other
      // waves go on to their tiles while the token waves build the tables
      // and reduce the virtual tiles (the gathers' latency hidden behind
      // the streaming waves).
      if (tok_wave && one_pass) {
        // pre[] by word runs; each thread ranks its own tokens, counts them,
        // penalises their logits (already in registers) and writes them by
        // rank (a token held twice writes the same values twice)
        GroupSync gs{&misc[M_GSYNC], TW, 0};
        const uint32_t U = build_pre(h, nwords, btot, TW, gs);
        LDS uint32_t* cnt = (LDS uint32_t*)h.pen;
        uint32_t rk[TQ];
#pragma unroll
        for (int q = 0; q < TQ; ++q) rk[q] = (tk[q] >= lo && tk[q] < hi) ? h.rank(tk[q]) : EMPTY;
        if (need_cnt) {
#pragma unroll
          for (int q = 0; q < TQ; ++q)
            if (rk[q] != EMPTY) __atomic_fetch_add(&cnt[rk[q]], umax(hc[q], 1u), __ATOMIC_RELAXED);
          gs();
        }
        float y[TQ];
#pragma unroll
        for (int q = 0; q < TQ; ++q) {
          y[q] = NEG_INF;
          if (rk[q] != EMPTY) {
            const bool allowed = (pm[q] >> (tk[q] & 31)) & 1u;
            const float x = pf[q];
            if (allowed && !(x < __builtin_huge_valf()) && P.mode == MODE_SAMPLE)
              __atomic_fetch_or(&misc[M_FLAGS], FLAG_NAN, __ATOMIC_RELAXED);
            float v = (x > NEG_INF) ? x : NEG_INF;  // NaN acts as -inf
            v = penalize(v, P, need_cnt ? cnt[rk[q]] : 1u);
            y[q] = allowed ? v : NEG_INF;
          }
        }
        if (need_cnt) gs();  // every count is read before pen[] (which holds them) is written
#pragma unroll
        for (int q = 0; q < TQ; ++q)
          if (rk[q] != EMPTY) {
            h.pen[rk[q]] = y[q];
            h.tokr[rk[q]] = tk[q];
          }
        gs();
        for (uint32_t k = (uint32_t)wv; k < nch; k += TW) vtile_chunk(a, t0, nwords, k, U, h, E, lane);
      } else if (tok_wave) {
        GroupSync gs{&misc[M_GSYNC], TW, 0};
        const uint32_t U = build_ranks(h, nwords, btot, &misc[M_FLAGS], TW, gs);
        if (need_cnt) {
          counts();
          gs();
        }
        if (ta != EMPTY) load_tile<DT>(a, row, mrow, h, ta, lane, ra);
#pragma unroll
        for (int q = 0; q < TQ; ++q) asm volatile("" ::"v"(pf[q]));  // the prefetch is done
        gather_penalised<DT>(a, P, b, row, U, h, need_cnt, TW, &misc[M_FLAGS]);
        gs();
        for (uint32_t k = (uint32_t)wv; k < nch; k += TW) vtile_chunk(a, t0, nwords, k, U, h, E, lane);
      }
    } else {
      BarrierSync bs;
      const uint32_t U = build_ranks(h, nwords, btot, &misc[M_FLAGS], NW, bs);
      if (need_cnt) {
        if (tok_wave) counts();
        __syncthreads();
      }
      gather_penalised<DT>(a, P, b, row, U, h, need_cnt, NW, &misc[M_FLAGS]);
      __syncthreads();
      for (uint32_t k = (uint32_t)wv; k < nch; k += NW) vtile_chunk(a, t0, nwords, k, U, h, E, lane);
    }
  }
  uint32_t since = EMPTY;

  auto process = [&](const Raw& raw, uint32_t t) __attribute__((always_inline)) {
    float v[16];
    unpack<DT>(raw, v);
    const uint32_t tb = t * TILE;
    if ((DT & SOFTCAP) && tb + TILE > a.V) {
      // positions past V hold -inf, which the cap would have made -cap
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if (tile_pos<DT>(tb, lane, j) >= a.V) v[j] = NEG_INF;
    }
    // history tokens and disallowed tokens become -inf (a uniform branch per
    // case, so a row without a mask spends nothing on one): a run's tokens
    // lie in one 32-bit word of the mask and of the bitmap
    constexpr int RUNS = (DT & 3) == LLMK_F32 ? 4 : 2, RL = 16 / RUNS;
    const uint32_t shr = (RL * (uint32_t)lane) & 31u;
    const uint32_t wl = (uint32_t)lane / (32u / RL);
    if (mrow) {
#pragma unroll
      for (int r = 0; r < RUNS; ++r) {
        uint32_t x = ~raw.mw[r];
        if (have) x |= h.bitmap[((tb - lo) >> 5) + (uint32_t)(8 * RL) * r / 4u + wl];
#pragma unroll
        for (int q = 0; q < RL; ++q) v[RL * r + q] = exclude(v[RL * r + q], x, shr + q);
      }
    } else if (have) {
#pragma unroll
      for (int r = 0; r < RUNS; ++r) {
        const uint32_t x = h.bitmap[((tb - lo) >> 5) + (uint32_t)(8 * RL) * r / 4u + wl];
#pragma unroll
        for (int q = 0; q < RL; ++q) v[RL * r + q] = exclude(v[RL * r + q], x, shr + q);
      }
    }
    tile_reduce(E, v, t, [&](int j) -> uint32_t { return tile_pos<DT>(tb, lane, j); }, since,
                lane);
  };
  // Later tiles are claimed dynamically, so the waves finish together.
  auto grab = [&]() -> uint32_t {
    uint32_t k = 0;
    if (lane == 0) k = __atomic_fetch_add(&misc[M_NEXT], 1u, __ATOMIC_RELAXED);
    k = (uint32_t)__builtin_amdgcn_readfirstlane((int)k);
    const uint32_t t = t0 + NW + k;
    return t < t1 ? t : EMPTY;
  };
  while (ta != EMPTY) {
    process(ra, ta);
    ta = grab();
    if (ta != EMPTY) load_tile<DT>(a, row, mrow, h, ta, lane, ra);
  }
  // ---- publish the segment; the row's last workgroup finalizes
  wait_stores();
  __syncthreads();
  if (tid == 0) {
    const uint32_t fl = misc[M_FLAGS];
    if (fl & FLAG_NAN) atomicOr(w.status, LLMK_STATUS_NAN_LOGITS);
    uint32_t last = 1;
    if (a.G > 1) {  // a single-segment row passes its table in registers
      G(w.seg_meta)[blockIdx.x] = u4v{misc[M_CCOUNT], misc[M_BETA], fl, have ? 1u : 0u};
      __threadfence();  // release this workgroup's stores (all waves waited above)
      const uint32_t old = atomicAdd(&w.row_arrive[b], 1u);
      last = (old == a.G - 1) ? 1u : 0u;
      if (last) {
        __threadfence();  // acquire the other segments' stores
        w.row_arrive[b] = 0;
      }
    }
    misc[M_LAST] = last;
  }
  __syncthreads();
  const uint32_t last = misc[M_LAST];
  const u4v seg_own = u4v{misc[M_CCOUNT], misc[M_BETA], misc[M_FLAGS], 0u};
  __syncthreads();  // finalize reuses this shared memory
  if (last) finalize_row<DT>(a, w, b, P, have, seg_own, u_row, sm);
}


// ===========================================================================
// Mask-form top-k and top-p (sampler.rs:160-216), in place on f32 rows
// ===========================================================================
// Order key with -0 folded onto +0: key order is then the order of `<` on
// every non-NaN value (the reference compares with `<`, sampler.rs:168).
__device__ __forceinline__ uint32_t ckey(float v) { return fkey(v == 0.0f ? 0.0f : v); }

constexpr uint32_t MK_BINS = 2048;  // 11-bit digits: key bits 31..21, 20..10, then 10 bits
constexpr uint32_t MK_CAP = NW * MK_BINS / 2;  // entries of the chosen bin gathered in LDS
constexpr uint32_t MK_LDS_WORDS = NW * MK_BINS + 512;

// Every element of row[e0..e1) once: float4 loads from the first 16-byte
// boundary on (lane-strided), single elements before it and after the last
// whole float4.  f(e, x) gets the first element's index and the values; the
// high bit of e marks a single element (in x.x).
template <class F>
__device__ __forceinline__ void each4(const float* row, uint32_t e0, uint32_t e1, F&& f) {
  const uint32_t mis = (uint32_t)(((uintptr_t)(row + e0) >> 2) & 3u);
  uint32_t a0 = e0 + (mis ? 4u - mis : 0u);
  if (a0 > e1) a0 = e1;
  const uint32_t v4 = a0 + ((e1 - a0) & ~3u);
  // four float4 loads in flight per lane before any is used: one workgroup
  // per row needs the memory-level parallelism
  constexpr uint32_t U = 4, STEP = 4 * NT;
  for (uint32_t e = a0 + 4 * threadIdx.x; e < v4; e += U * STEP) {
    f4v x[U];
#pragma unroll
    for (uint32_t u = 0; u < U; ++u)
      if (e + u * STEP < v4) x[u] = *(const GLB f4v*)G(row + e + u * STEP);
#pragma unroll
    for (uint32_t u = 0; u < U; ++u)
      if (e + u * STEP < v4) f(e + u * STEP, x[u]);
  }
  const uint32_t nh = a0 - e0, ns = nh + (e1 - v4);
  for (uint32_t i = threadIdx.x; i < ns; i += NT) {
    const uint32_t e = i < nh ? e0 + i : v4 + (i - nh);
    f4v x;
    x.x = G(row)[e];
    x.y = x.z = x.w = NEG_INF;
    f(e | 0x80000000u, x);
  }
}

// apply_top_k in one read of the row (top_k <= MK1_KMAX, V <= MK1_VMAX):
// every value at or above a rising threshold is gathered into LDS as it is
// read, the threshold being the lower edge of the top_k-th largest fine bin
// (key >> 20) of what has been counted so far -- the first round of the
// workgroup (16 values per thread) is counted whole before any is gathered,
// later gathers count themselves -- so it only rises and never passes the
// true top_k-th largest value tau: every value
// >= tau is gathered, and the top_k-th largest gathered value is tau.  The
// kept positions (values >= tau, and NaN, which `v < threshold` never
// masks) go into an LDS bitmap, and a second pass only writes: -inf over
// every position not kept.  Returns false, having written nothing, when the
// gathered values overflow the buffer (then the radix select runs).
constexpr uint32_t MK1_CAP = 8192;       // gathered values
constexpr uint32_t MK1_NAN = 256;        // gathered NaN positions
constexpr uint32_t MK1_KMAX = 1024;
constexpr uint32_t MK1_VMAX = 1u << 18;  // the kept bitmap's reach
constexpr uint32_t MK1_LDS_WORDS = NBINS + 64 + 64 + MK1_VMAX / 32 + 2 * MK1_CAP + MK1_NAN;
static_assert(MK1_LDS_WORDS <= MK_LDS_WORDS, "the one-read path fits the kernel's shared memory");
__device__ __forceinline__ bool topk_one_read(float* row, uint32_t V, uint32_t K,
                                              LDS uint32_t* smem) {
  const uint32_t tid = threadIdx.x;
  const int lane = (int)(tid & 63u);
  LDS uint32_t* hf = smem;             // NBINS fine bins (key >> 20)
  LDS uint32_t* hc = hf + NBINS;       // 64 coarse bins (key >> 26)
  LDS uint32_t* sc = hc + 64;          // [0] gathered, [1] beta, [2] NaNs, [3] flags
  LDS uint32_t* bm = sc + 64;          // kept bitmap, (V + 31) / 32 words
  LDS float* cval = (LDS float*)(bm + MK1_VMAX / 32);
  LDS uint32_t* cidx = (LDS uint32_t*)(cval + MK1_CAP);
  LDS uint32_t* nidx = cidx + MK1_CAP;
  const uint32_t nwords = (V + 31) / 32;
  for (uint32_t i = tid; i < NBINS; i += NT) hf[i] = 0;
  for (uint32_t i = tid; i < nwords; i += NT) bm[i] = 0;
  if (tid < 64) hc[tid] = 0;
  if (tid < 4) sc[tid] = 0;
  __syncthreads();
  // the float4-aligned body [a0, v4) in rounds of U float4 per thread, and
  // the single elements before and after it
  const uint32_t mis = (uint32_t)(((uintptr_t)row >> 2) & 3u);
  const uint32_t a0 = umin(mis ? 4u - mis : 0u, V);
  const uint32_t v4 = a0 + ((V - a0) & ~3u);
  constexpr uint32_t U = 4, STEP = 4 * NT;
  const uint32_t nrounds = (v4 - a0 + U * STEP - 1) / (U * STEP);
  auto gather = [&](float v, uint32_t e, uint32_t thr, bool count) __attribute__((always_inline)) {
    if (v != v) {
      const uint32_t at = __atomic_fetch_add(&sc[2], 1u, __ATOMIC_RELAXED);
      if (at < MK1_NAN) nidx[at] = e;
      return;
    }
    const uint32_t key = ckey(v);
    if (key < thr) return;
    const uint32_t at = __atomic_fetch_add(&sc[0], 1u, __ATOMIC_RELAXED);
    if (at < MK1_CAP) {
      cval[at] = v == 0.0f ? 0.0f : v;
      cidx[at] = e;
    }
    if (count) {
      __atomic_fetch_add(&hf[key >> BIN_SHIFT], 1u, __ATOMIC_RELAXED);
      __atomic_fetch_add(&hc[key >> CBIN_SHIFT], 1u, __ATOMIC_RELAXED);
    }
  };
  // the singles first (gathered at threshold 0, counted in the fine bins:
  // the first round's coarse sums include them)
  const uint32_t ns = a0 + (V - v4);
  for (uint32_t i = tid; i < ns; i += NT) {
    const uint32_t e = i < a0 ? i : v4 + (i - a0);
    const float v = G(row)[e];
    gather(v, e, 0u, false);
    if (v > NEG_INF && v == v) __atomic_fetch_add(&hf[ckey(v) >> BIN_SHIFT], 1u, __ATOMIC_RELAXED);
  }
  __syncthreads();
  for (uint32_t r = 0; r < nrounds; ++r) {
    f4v x[U];
    const uint32_t eb = a0 + 4 * tid + r * U * STEP;
#pragma unroll
    for (uint32_t u = 0; u < U; ++u)
      x[u] = eb + u * STEP < v4 ? __builtin_nontemporal_load((const GLB f4v*)G(row + eb + u * STEP))
                                : f4v{NEG_INF, NEG_INF, NEG_INF, NEG_INF};
    if (r == 0) {
      // the first round: every value counted in the fine bins, the coarse
      // bins summed from them, the threshold raised; the round is then
      // gathered without counting again
#pragma unroll
      for (uint32_t u = 0; u < U; ++u) {
        const float vv[4] = {x[u].x, x[u].y, x[u].z, x[u].w};
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (vv[q] > NEG_INF && vv[q] == vv[q])
            __atomic_fetch_add(&hf[ckey(vv[q]) >> BIN_SHIFT], 1u, __ATOMIC_RELAXED);
      }
      __syncthreads();
      if (tid < 64) {
        uint32_t c = 0;
        for (uint32_t i = 0; i < 64; ++i) c += hf[64 * tid + i];
        hc[tid] = c;
      }
      __syncthreads();
      if (tid < 64) {
        const uint32_t nb = compute_beta(hc, hf, K, lane);
        if (lane == 0) sc[1] = nb;
      }
      __syncthreads();
    }
    uint32_t beta = __atomic_load_n(&sc[1], __ATOMIC_RELAXED);
    const uint32_t thr = beta << BIN_SHIFT;
    bool any = false;
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) {
      const uint32_t e = eb + u * STEP;
      if (e >= v4) continue;
      const float vv[4] = {x[u].x, x[u].y, x[u].z, x[u].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const bool hit = !(ckey(vv[q]) < thr) || vv[q] != vv[q];
        any |= hit;
        if (hit) gather(vv[q], e + q, thr, r > 0);
      }
    }
    if (r > 0 && __ballot(any)) {
      const uint32_t nb = compute_beta(hc, hf, K, lane);
      if (nb > beta && lane == 0) __atomic_fetch_max(&sc[1], nb, __ATOMIC_RELAXED);
    }
  }
  __syncthreads();
  const uint32_t n = sc[0], nn = sc[2];
  if (n > MK1_CAP || nn > MK1_NAN || n < K) return false;
  __syncthreads();  // every thread has read the counts before sc is reused
  const uint32_t tau = kth_largest_key<BlockSync>(cval, n, K, hf, sc + 8);
  for (uint32_t i = tid; i < n; i += NT)
    if (ckey(cval[i]) >= tau) __atomic_fetch_or(&bm[cidx[i] >> 5], 1u << (cidx[i] & 31u), __ATOMIC_RELAXED);
  for (uint32_t i = tid; i < nn; i += NT)
    __atomic_fetch_or(&bm[nidx[i] >> 5], 1u << (nidx[i] & 31u), __ATOMIC_RELAXED);
  __syncthreads();
  // write only: -inf wherever nothing is kept (kept values stay as they are)
  for (uint32_t i = tid; i < ns; i += NT) {
    const uint32_t e = i < a0 ? i : v4 + (i - a0);
    if (!((bm[e >> 5] >> (e & 31u)) & 1u)) G(row)[e] = NEG_INF;
  }
  for (uint32_t e = a0 + 4 * tid; e < v4; e += STEP) {
    // the four positions' bits (e is 16-byte aligned in memory, not a
    // multiple of 4 when the row is not: they may straddle two words)
    const uint32_t w = e >> 5, sh = e & 31u;
    const uint32_t kb = (uint32_t)((((uint64_t)(sh > 28u ? bm[w + 1] : 0u) << 32) | bm[w]) >> sh) & 15u;
    if (kb == 0) {
      __builtin_nontemporal_store(f4v{NEG_INF, NEG_INF, NEG_INF, NEG_INF}, (GLB f4v*)G(row + e));
    } else {
#pragma unroll
      for (uint32_t q = 0; q < 4; ++q)
        if (!((kb >> q) & 1u)) G(row)[e + q] = NEG_INF;
    }
  }
  return true;
}

// apply_top_k (sampler.rs:160-173) for one row per workgroup: the key of
// the top_k-th largest value by a radix select over the row (11-bit digits
// counted in per-wave LDS histograms), stopping once the chosen digit holds
// at most MK_CAP values; those are gathered into LDS and the select ends
// there, while the same pass masks every value whose key prefix lies below.
__global__ __launch_bounds__(NT) void topk_mask_kernel(float* logits, uint32_t V,
                                                       uint64_t stride,
                                                       const int32_t* top_k) {
  extern __shared__ __align__(16) uint32_t smem[];
  const uint32_t b = blockIdx.x, tid = threadIdx.x;
  const uint32_t wv = tid >> 6;
  const int32_t k = G(top_k)[b];
  if (k <= 0 || (uint32_t)k >= V) return;  // sampler.rs:161-163
  float* row = logits + (uint64_t)b * stride;
  if ((uint32_t)k <= MK1_KMAX && V <= MK1_VMAX &&
      topk_one_read(row, V, (uint32_t)k, (LDS uint32_t*)smem))
    return;
  __syncthreads();  // the radix select reuses the shared memory
  LDS uint32_t* hist = (LDS uint32_t*)smem;  // NW * MK_BINS
  LDS uint32_t* sh = hist + NW * MK_BINS;     // 512: select histogram, scalars
  uint32_t pbits = 0, pref = 0, need = (uint32_t)k, cnt = V;
  while (pbits < 32 && cnt > MK_CAP) {
    const uint32_t dbits = pbits == 22 ? 10u : 11u;
    const uint32_t shift = 32 - pbits - dbits, dmask = (1u << dbits) - 1u;
    for (uint32_t i = tid; i < NW * MK_BINS; i += NT) hist[i] = 0;
    __syncthreads();
    LDS uint32_t* wh = hist + wv * MK_BINS;
    each4(row, 0, V, [&](uint32_t e, f4v x) {
      const float vv[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (q > 0 && (e & 0x80000000u)) break;
        const uint32_t key = ckey(vv[q]);
        if (pbits == 0 || (key >> (32 - pbits)) == pref)
          __atomic_fetch_add(&wh[(key >> shift) & dmask], 1u, __ATOMIC_RELAXED);
      }
    });
    __syncthreads();
    // thread t: digits 2047 - 2t and 2046 - 2t (descending), summed over waves
    uint32_t c2[2] = {0u, 0u};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t d = MK_BINS - 1 - 2 * tid - j;
      for (uint32_t w2 = 0; w2 < NW; ++w2) c2[j] += hist[w2 * MK_BINS + d];
    }
    uint32_t total;
    const uint32_t above = block_excl_scan(c2[0] + c2[1], sh + 256, total);
    if (above < need && above + c2[0] + c2[1] >= need) {
      const bool first = above + c2[0] >= need;
      const uint32_t d = MK_BINS - 1 - 2 * tid - (first ? 0 : 1);
      sh[300] = d & dmask;
      sh[301] = need - above - (first ? 0 : c2[0]);
      sh[302] = first ? c2[0] : c2[1];
    }
    __syncthreads();
    pref = (pref << dbits) | sh[300];
    pbits += dbits;
    need = sh[301];
    cnt = sh[302];
    __syncthreads();
  }
  // Final pass: values whose key prefix is below pref are below the
  // threshold; with pbits == 32 the threshold is known and the rest stay,
  // otherwise the cnt values of prefix pref are gathered for the last select.
  LDS float* cval = (LDS float*)hist;
  LDS uint32_t* cidx = hist + MK_CAP;
  if (tid == 0) sh[303] = 0;
  __syncthreads();
  const uint32_t pshift = 32 - pbits;
  each4(row, 0, V, [&](uint32_t e, f4v x) {
    const bool one = (e & 0x80000000u) != 0;
    const uint32_t e0 = e & 0x7fffffffu;
    float vv[4] = {x.x, x.y, x.z, x.w};
    bool dirty = false;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (q > 0 && one) break;
      const float v = vv[q];
      if (v != v) continue;  // NaN: `v < threshold` is false
      const uint32_t kp = pshift == 32 ? 0u : ckey(v) >> pshift;
      if (kp < pref) {
        if (v != NEG_INF) {
          vv[q] = NEG_INF;
          dirty = true;
        }
      } else if (kp == pref && pbits < 32) {
        const uint32_t at = __atomic_fetch_add(&sh[303], 1u, __ATOMIC_RELAXED);
        if (at < MK_CAP) {
          cval[at] = v == 0.0f ? 0.0f : v;
          cidx[at] = e0 + q;
        }
      }
    }
    if (dirty) {
      if (one) G(row)[e0] = vv[0];
      else *(GLB f4v*)G(row + e0) = f4v{vv[0], vv[1], vv[2], vv[3]};
    }
  });
  if (pbits == 32) return;
  // the float4 stores above may cover gathered entries masked below
  wait_stores();
  __syncthreads();
  const uint32_t n = sh[303] < MK_CAP ? sh[303] : MK_CAP;  // cnt less the NaNs
  if (n == 0) return;
  const float thr =
      funkey(kth_largest_key<BlockSync>(cval, n, need < n ? need : n, sh, sh + 304));
  for (uint32_t i = tid; i < n; i += NT)
    if (cval[i] < thr) G(row)[cidx[i]] = NEG_INF;
}

// The last key k in [lo, hi) with pred(k), given pred(lo) and !pred(hi),
// pred true then false over [lo, hi]: a 64-way search by one wave, six
// rounds for 32-bit keys (bounded to eight).
template <class P>
__device__ __forceinline__ uint32_t band_edge(uint32_t lo, uint32_t hi, int lane, P&& pred) {
  for (int it = 0; it < 8 && hi - lo > 1u; ++it) {
    const uint32_t step = (hi - lo + 63u) / 64u;
    const uint64_t kj = (uint64_t)lo + (uint64_t)step * (uint32_t)lane;
    const bool in = lane > 0 && kj < hi;
    const bool t = in && pred((uint32_t)kj);
    const uint64_t mi = __ballot(in), mf = __ballot(in && !t);
    if (mf) {
      const uint32_t f = (uint32_t)__ffsll((long long)mf) - 1u;  // >= 1
      hi = lo + step * f;
      lo = lo + step * (f - 1u);
    } else {
      lo = lo + step * (uint32_t)(63 - __clzll((long long)mi));
    }
  }
  return lo;
}

// apply_top_p (sampler.rs:176-216) after the sampling kernel has found the
// row's cut with the same probabilities (temperature 1, nothing else): the
// kept prefix, in (p desc, index asc) order, ends at token c of probability
// p_c.  p is non-decreasing in the value, so the values of probability p_c
// form one key interval [klo, khi], found by two 64-way searches in wave 0;
// a value is kept if its key is above khi, or within the interval at an
// index <= c.  Grid: rows x segments of seg elements.
__global__ __launch_bounds__(NT) void topp_mask_kernel(float* logits, uint32_t V,
                                                       uint64_t stride, const float* top_p,
                                                       const u4v* cut, const uint32_t* tok,
                                                       uint32_t nseg, uint32_t seg) {
  __shared__ uint32_t band[4];
  const uint32_t b = blockIdx.x / nseg, g = blockIdx.x % nseg;
  const uint32_t tid = threadIdx.x;
  const int lane = (int)(tid & 63);
  float* row = logits + (uint64_t)b * stride;
  exp_tab_init();
  __syncthreads();
  if (tid < WAVE) {
    const float tp = G(top_p)[b];
    const u4v r = G(cut)[b];
    const uint32_t t = G(tok)[b];
    const float m = __uint_as_float(r.z), S = __uint_as_float(r.w);
    // no-op rows: top_p >= 1 or NaN (sampler.rs:177-179), softmax sum 0
    // (sampler.rs:190-192), everything kept (the cut never reached), or the
    // sampling kernel could not serve the row
    bool run = tp < 1.0f && t != LLMK_INVALID_TOKEN && r.y < V && S > 0.0f && r.x < V;
    uint32_t klo = 0, khi = 0;
    if (run) {
      const float pc = prob_of(G(row)[r.x], 1.0f, m, S);
      const uint32_t kc = ckey(G(row)[r.x]);
      auto pk = [&](uint32_t key) { return prob_of(funkey(key), 1.0f, m, S); };
      // khi: the last key with p <= pc, in [kc, key(m)]
      const uint32_t km = ckey(m);
      khi = (km <= kc || !(pk(km) > pc))
                ? 0xffffffffu
                : band_edge(kc, km, lane, [&](uint32_t key) { return pk(key) <= pc; });
      // klo: the first key with p >= pc, in (key(-inf), kc]: p(-inf) = 0 < pc
      klo = 1u + band_edge(0x007fffffu, kc, lane, [&](uint32_t key) { return pk(key) < pc; });
    }
    if (lane == 0) {
      band[0] = run ? 1u : 0u;
      band[1] = klo;
      band[2] = khi;
      band[3] = r.x;
    }
  }
  __syncthreads();
  if (!band[0]) return;
  const uint32_t klo = band[1], khi = band[2], c = band[3];
  const uint32_t e0 = g * seg, e1 = e0 + seg < V ? e0 + seg : V;
  each4(row, e0, e1, [&](uint32_t e, f4v x) {
    const bool one = (e & 0x80000000u) != 0;
    const uint32_t ea = e & 0x7fffffffu;
    float vv[4] = {x.x, x.y, x.z, x.w};
    bool dirty = false;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (q > 0 && one) break;
      const float v = vv[q];
      const uint32_t key = ckey(v);
      const bool keep = key > khi || (key >= klo && ea + q <= c);
      if (!keep && v != NEG_INF) {
        vv[q] = NEG_INF;
        dirty = true;
      }
    }
    if (dirty) {
      if (one) G(row)[ea] = vv[0];
      else *(GLB f4v*)G(row + ea) = f4v{vv[0], vv[1], vv[2], vv[3]};
    }
  });
}


// Logit bias in place (the formula of llm-tests/tests/mlc_parity.rs:1060-1072,
// l += bias): one wave per row, lanes over the row's (token, bias) list.
// The add is a compare-and-swap loop, an IEEE f32 addition (denormals kept)
// that keeps both biases of a token listed twice; each round one of the
// contending lanes succeeds, so the loop ends.
__global__ __launch_bounds__(NT) void logit_bias_kernel(float* logits, uint32_t B, uint32_t V,
                                                        uint64_t stride, const uint32_t* off,
                                                        const uint32_t* tok, const float* val) {
  const uint32_t b = blockIdx.x * NW + (threadIdx.x >> 6);
  if (b >= B) return;
  const uint32_t j0 = G(off)[b], j1 = G(off)[b + 1];
  for (uint32_t j = j0 + (threadIdx.x & 63u); j < j1; j += WAVE) {
    const uint32_t t = G(tok)[j];
    if (t < V) {
      uint32_t* p = (uint32_t*)(logits + (uint64_t)b * stride + t);
      const float v = G(val)[j];
      uint32_t old = G(p)[0], seen;
      do {
        seen = old;
        old = atomicCAS(p, seen, __float_as_uint(__uint_as_float(seen) + v));
      } while (old != seen);
    }
  }
}


// The scheduler's token push (scheduler.rs:147) on the device: row b appends
// its sampled token to its history buffer, htok[hoff[b] + hlen[b]], while
// hlen[b] < cap.  A full row keeps its history and raises a status bit.
__global__ __launch_bounds__(256) void history_append_kernel(uint32_t B, const uint32_t* hoff,
                                                             uint32_t* hlen, uint32_t* htok,
                                                             uint32_t cap, const uint32_t* tok,
                                                             uint32_t* status) {
  const uint32_t b = blockIdx.x * 256 + threadIdx.x;
  if (b >= B) return;
  const uint32_t t = G(tok)[b];
  if (t == LLMK_INVALID_TOKEN) return;
  const uint32_t n = G(hlen)[b];
  if (n >= cap) {
    atomicOr(status, LLMK_STATUS_HISTORY_FULL);
    return;
  }
  G(htok)[G(hoff)[b] + n] = t;
  G(hlen)[b] = n + 1;
}

// The count-table form of the same push: row b's history is its distinct
// tokens htok[hoff[b] .. hoff[b] + hlen[b]) in ascending order, with their
// occurrences in hcnt at the same positions.  A token already listed has its
// count raised by one; a new one is inserted in order with count 1 (the
// entries above it move up by one) while hlen[b] < cap, else the row keeps
// its table and raises a status bit.  One workgroup per row: its entries are
// read HCA_Q per thread, below-t counted and an equal entry looked for, then
// the entries from the insertion point up are moved, the highest chunk
// first, every read of a chunk before any of its writes.
constexpr uint32_t HCA_T = 256, HCA_Q = 8, HCA_CH = HCA_T * HCA_Q;
__global__ __launch_bounds__(HCA_T) void history_count_append_kernel(
    const uint32_t* hoff, uint32_t* hlen, uint32_t* htok, uint32_t* hcnt, uint32_t cap,
    const uint32_t* tok, uint32_t* status) {
  __shared__ uint32_t red[2 * (HCA_T / WAVE)];
  const uint32_t b = blockIdx.x, tid = threadIdx.x, lane = tid & 63u, wv = tid >> 6;
  const uint32_t t = G(tok)[b];
  if (t == LLMK_INVALID_TOKEN) return;
  const uint32_t off = G(hoff)[b], n = G(hlen)[b];
  GLB uint32_t* T = G(htok) + off;
  GLB uint32_t* C = G(hcnt) + off;
  uint32_t below = 0, eq = EMPTY;
  for (uint32_t c0 = 0; c0 < n; c0 += HCA_CH) {
    uint32_t x[HCA_Q];
#pragma unroll
    for (uint32_t q = 0; q < HCA_Q; ++q) {
      const uint32_t i = c0 + q * HCA_T + tid;
      x[q] = i < n ? T[i] : EMPTY;
    }
#pragma unroll
    for (uint32_t q = 0; q < HCA_Q; ++q) {
      const uint32_t i = c0 + q * HCA_T + tid;
      if (i < n) {
        below += x[q] < t ? 1u : 0u;
        if (x[q] == t) eq = umin(eq, i);
      }
    }
  }
  below = bcast63u(wave_incl_scan(below));
  eq = wave_min_u32(eq);
  if (lane == 0) {
    red[wv] = below;
    red[HCA_T / WAVE + wv] = eq;
  }
  __syncthreads();
  below = 0;
  eq = EMPTY;
#pragma unroll
  for (uint32_t i = 0; i < HCA_T / WAVE; ++i) {
    below += red[i];
    eq = umin(eq, red[HCA_T / WAVE + i]);
  }
  if (eq != EMPTY) {
    // a listed count of 0 reads as 1 occurrence (hist_weight): one more is 2
    if (tid == 0) C[eq] = umax(C[eq], 1u) + 1u;
    return;
  }
  if (n >= cap) {
    if (tid == 0) atomicOr(status, LLMK_STATUS_HISTORY_FULL);
    return;
  }
  const uint32_t pos = below;
  for (uint32_t hi = n; hi > pos;) {
    const uint32_t lo = hi - pos > HCA_CH ? hi - HCA_CH : pos;
    uint32_t xt[HCA_Q], xc[HCA_Q];
#pragma unroll
    for (uint32_t q = 0; q < HCA_Q; ++q) {
      const uint32_t i = lo + q * HCA_T + tid;
      xt[q] = i < hi ? T[i] : 0u;
      xc[q] = i < hi ? C[i] : 0u;
    }
    __syncthreads();  // the chunk's reads before its writes (the next chunk's reads lie below lo)
#pragma unroll
    for (uint32_t q = 0; q < HCA_Q; ++q) {
      const uint32_t i = lo + q * HCA_T + tid;
      if (i < hi) {
        T[i + 1] = xt[q];
        C[i + 1] = xc[q];
      }
    }
    hi = lo;
  }
  __syncthreads();  // entry pos was read by the first chunk before it is rewritten
  if (tid == 0) {
    T[pos] = t;
    C[pos] = 1u;
    G(hlen)[b] = n + 1u;
  }
}

// ---------------------------------------------------------------------------
// Speculative-decoding verification (docs/mlc-contracts.md:83-84: accept the
// draft token unless r >= p/q, else resample from max(p - q, 0))
// ---------------------------------------------------------------------------
struct VerifyArgs {
  uint32_t B, V, cap;      // rows, vocabulary, list stride (the sampler's out_cap)
  const uint32_t* ids;     // [B][cap]: the target's kept ids, (p desc, idx asc)
  const float* probs;      // [B][cap]: their processed probabilities
  const uint32_t* cnt;     // [B]: kept counts
  const uint32_t* draft;   // [B]: draft tokens
  const float* q;          // [B][qstride]: the draft distribution over the vocabulary
  uint64_t qstride;
  const float* ua;         // [B]: uniforms of the acceptance test
  const float* ur;         // [B]: uniforms of the residual draw
  uint32_t* out_tok;       // [B]
  uint32_t* out_acc;       // [B]: 1 accepted, 0 resampled
};

// The residual max(p_i - q[id_i], 0) of kept entry i (one f32 subtraction),
// through the divisor chain: the list the residual draw scans, in the
// target's (p desc, idx asc) order.
struct ResidualList {
  const float* p;
  const uint32_t* idx;
  const float* q;
  uint32_t V;  // an id at or above V (not one the sampler writes) reads q = 0
  Chain c;
  __device__ float raw(uint32_t i) const {
    const uint32_t t = G(idx)[i];
    const float r = G(p)[i] - (t < V ? G(q)[t] : 0.0f);
    return r > 0.0f ? r : 0.0f;
  }
  __device__ float get(uint32_t i) const { return c.apply(raw(i)); }
};

// One wave per row.  Accept when u_a * q(d) < p(d) (the draft token d's
// target probability p(d) is 0 outside the kept list).  Otherwise the
// residual sum R is the sequential f32 sum of the residuals in list order,
// and the token is the reference's draw (sampler.rs:113-124) over the
// residuals divided by R: the first entry whose running sum reaches u_r, else
// the last entry with a positive residual.  R = 0 (p <= q on every kept
// entry) draws from p itself.  A row whose list is empty or was cut short
// (count > cap), or whose draft token is not below V, is invalid.
__global__ __launch_bounds__(WAVE) void verify_kernel(VerifyArgs v, uint32_t* status) {
  __shared__ uint32_t sh_[2];
  __shared__ float z_[2 * WAVE];
  LDS uint32_t* sh = (LDS uint32_t*)sh_;
  LDS float* z = (LDS float*)z_;
  const uint32_t b = blockIdx.x, lane = threadIdx.x;
  const uint32_t n = G(v.cnt)[b], d = G(v.draft)[b];
  if (n == 0 || n > v.cap || d >= v.V) {
    if (lane == 0) {
      G(v.out_tok)[b] = LLMK_INVALID_TOKEN;
      G(v.out_acc)[b] = 0u;
      atomicOr(status, LLMK_STATUS_INVALID_PARAMS);
    }
    return;
  }
  const uint32_t* ids = v.ids + (uint64_t)b * v.cap;
  const float* probs = v.probs + (uint64_t)b * v.cap;
  const float* q = v.q + (uint64_t)b * v.qstride;
  uint32_t jd = EMPTY;  // ids are distinct: at most one entry holds d
  for (uint32_t j = lane; j < n; j += WAVE)
    if (G(ids)[j] == d) jd = j;
  jd = wave_min_u32(jd);
  const float pd = jd < n ? G(probs)[jd] : 0.0f;
  const float qd = G(q)[d];
  const float ua = G(v.ua)[b], ur = G(v.ur)[b];
  uint32_t tok = d, acc = 1u;
  if (!(ua * qd < pd)) {
    acc = 0u;
    ResidualList rl{probs, ids, q, v.V, Chain{0.0f, 0.0f, 0.0f, 0}};
    float R;
    seq_scan(rl, n, 0, 0.0f, R, sh, z);
    float c;
    if (R > 0.0f) {
      rl.c.push(R);
      const uint32_t j = seq_scan(rl, n, 2, ur, c, sh, z);
      if (j < n) {
        tok = G(ids)[j];
      } else {
        uint32_t jl = 0;  // the last entry with a positive residual (R > 0: one exists)
        for (uint32_t i = lane; i < n; i += WAVE)
          if (rl.raw(i) > 0.0f) jl = i + 1;
        jl = wave_max_u32(jl);
        tok = G(ids)[jl - 1];
      }
    } else {
      List pl{probs, ids, Chain{0.0f, 0.0f, 0.0f, 0}, nullptr};
      const uint32_t j = seq_scan(pl, n, 2, ur, c, sh, z);
      tok = G(ids)[j < n ? j : n - 1];
    }
  }
  if (lane == 0) {
    G(v.out_tok)[b] = tok;
    G(v.out_acc)[b] = acc;
  }
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
  void* stage;         // aligned copies of rows passed at any offset (allocated on demand)
  size_t stage_bytes;
  uint32_t epoch;      // calls made (their parity picks the job count)
  uint32_t ncu;        // the device's compute units
  uint32_t xs_spin;    // phase 1's wait limit (LLMK_TEST_XS_SPIN at create, for tests)
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

static constexpr size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Dynamic LDS of one workgroup: the CU's 160 KiB less the kernels' static
// LDS (the expf table, the phase words and the copy of the arguments for the
// finalize's rare paths, under 1 KiB).
static_assert(sizeof(KCtx) + 32 * 8 + 4 * 4 + 2 * 4 < 1024, "static LDS above 1 KiB");
static constexpr size_t LDS_DYN_MAX = 160 * 1024 - 1024;

// The workspace of the sampling kernel for batches up to mb rows of up to mv
// logits, pool workgroup entries and `slots` slow-path slots: byte offsets
// of its arrays in one 256-byte aligned block.
struct WsLayout {
  size_t arrive, part, meta, cand, lock, skeys, sp, si, status, cut, mtok, zu;
  size_t xctl, xjob, xwsum, xwflag, xmeta, xterms, xruns, xsave, total;
};
static constexpr uint32_t xs_maxw(uint32_t mv) { return (mv + XS_W - 1) / XS_W; }
static constexpr WsLayout ws_layout(uint32_t mb, uint32_t mv, uint32_t pool, uint32_t slots) {
  WsLayout L{};
  size_t off = 0;
  L.arrive = off; off = align_up(off + 4ull * mb, 256);
  L.part = off; off = align_up(off + 8ull * mb * MAX_SLOTS, 256);
  L.meta = off; off = align_up(off + 16ull * pool, 256);
  L.cand = off; off = align_up(off + 8ull * pool * CAND_CAP, 256);
  L.lock = off; off = align_up(off + 4ull * slots, 256);
  L.skeys = off; off = align_up(off + 8ull * slots * 3 * mv, 256);
  L.sp = off; off = align_up(off + 4ull * slots * mv, 256);
  L.si = off; off = align_up(off + 4ull * slots * mv, 256);
  L.status = off; off = align_up(off + 256, 256);
  L.cut = off; off = align_up(off + 16ull * mb, 256);
  L.mtok = off; off = align_up(off + 4ull * mb, 256);
  L.zu = off; off = align_up(off + 4ull * mb, 256);
  const uint64_t mw = xs_maxw(mv);
  L.xctl = off; off = align_up(off + 4ull * XS_CTL_WORDS, 256);
  L.xjob = off; off = align_up(off + 4ull * XS_JOBS * XS_JOB_WORDS, 256);
  L.xwsum = off; off = align_up(off + 4ull * XS_JOBS * mw, 256);
  L.xwflag = off; off = align_up(off + 4ull * XS_JOBS * mw, 256);
  L.xmeta = off; off = align_up(off + 4ull * XS_JOBS * mw * 16 * 8, 256);
  L.xterms = off; off = align_up(off + 4ull * XS_JOBS * mw * 16 * TILE, 256);
  L.xruns = off; off = align_up(off + 4ull * XS_JOBS * mw * 16 * XS_RUNW, 256);
  L.xsave = off; off = align_up(off + 4ull * XS_JOBS * XS_SAVE, 256);
  L.total = off;
  return L;
}
static Ws ws_carve(char* base, const WsLayout& L, uint32_t mv, uint32_t slots) {
  Ws w;
  w.row_arrive = (uint32_t*)(base + L.arrive);
  w.tile_part = (f2v*)(base + L.part);
  w.seg_meta = (u4v*)(base + L.meta);
  w.cand = (u2v*)(base + L.cand);
  w.slow_lock = (uint32_t*)(base + L.lock);
  w.slow_keys = (uint64_t*)(base + L.skeys);
  w.slow_p = (float*)(base + L.sp);
  w.slow_idx = (uint32_t*)(base + L.si);
  w.status = (uint32_t*)(base + L.status);
  w.cut = (u4v*)(base + L.cut);
  w.mtok = (uint32_t*)(base + L.mtok);
  w.zu = (float*)(base + L.zu);
  w.xs_ctl = (uint32_t*)(base + L.xctl);
  w.xs_job = (uint32_t*)(base + L.xjob);
  w.xs_wsum = (float*)(base + L.xwsum);
  w.xs_wflag = (uint32_t*)(base + L.xwflag);
  w.xs_meta = (uint32_t*)(base + L.xmeta);
  w.xs_terms = (float*)(base + L.xterms);
  w.xs_runs = (uint32_t*)(base + L.xruns);
  w.xs_save = (uint32_t*)(base + L.xsave);
  w.xs_maxw = xs_maxw(mv);
  w.max_vocab = mv;
  w.slow_slots = slots;
  return w;
}
// Dynamic LDS above 64 KiB must be allowed explicitly (per device; no
// allocation).
static int set_kernel_attributes() {
  const void* kernels[] = {
      (const void*)stream_kernel<LLMK_F32>,           (const void*)stream_kernel<LLMK_BF16>,
      (const void*)stream_kernel<LLMK_F16>,           (const void*)stream_kernel<LLMK_F32 | SOFTCAP>,
      (const void*)stream_kernel<LLMK_BF16 | SOFTCAP>, (const void*)stream_kernel<LLMK_F16 | SOFTCAP>,
      (const void*)xs_kernel<LLMK_F32>,               (const void*)xs_kernel<LLMK_BF16>,
      (const void*)xs_kernel<LLMK_F16>,               (const void*)xs_kernel<LLMK_F32 | SOFTCAP>,
      (const void*)xs_kernel<LLMK_BF16 | SOFTCAP>,     (const void*)xs_kernel<LLMK_F16 | SOFTCAP>};
  for (const void* k : kernels)
    HIPCHK(hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, LDS_DYN_MAX));
  HIPCHK(hipFuncSetAttribute((const void*)topk_mask_kernel,
                             hipFuncAttributeMaxDynamicSharedMemorySize, 4 * MK_LDS_WORDS));
  return LLMK_OK;
}

extern "C" int llmk_sampler_create(llmk_sampler** out, int device,
                                   uint32_t max_batch, uint32_t max_vocab) {
  if (!out) return fail(LLMK_ERR_INVALID_ARGUMENT, "out is NULL");
  *out = nullptr;
  if (max_batch == 0 || max_vocab == 0)
    return fail(LLMK_ERR_INVALID_ARGUMENT, "max_batch and max_vocab must be > 0");
  if (max_vocab > MAX_TILES * TILE)
    return fail(LLMK_ERR_CAPACITY, "max_vocab above 2^20");
  if (4 * slow_lds_words(max_vocab) > LDS_DYN_MAX)
    return fail(LLMK_ERR_CAPACITY, "max_vocab too large for the slow path's LDS tables");
  HIPCHK(hipSetDevice(device));
  const int rc = set_kernel_attributes();
  if (rc != LLMK_OK) return rc;
  const uint32_t pool = max_batch > MAX_WGS ? max_batch : MAX_WGS;
  const uint32_t slots = max_batch < SLOW_SLOTS ? max_batch : SLOW_SLOTS;
  const WsLayout L = ws_layout(max_batch, max_vocab, pool, slots);
  void* mem = nullptr;
  HIPCHK(hipMalloc(&mem, L.total));
  hipError_t e = hipMemset(mem, 0, L.total);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    (void)hipFree(mem);
    return fail(LLMK_ERR_HIP, std::string("workspace init failed: ") + hipGetErrorString(e));
  }
  llmk_sampler* s = new llmk_sampler();
  s->device = device;
  s->max_batch = max_batch;
  s->max_vocab = max_vocab;
  int ncu = 0;
  if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
    ncu = 0;  // phase 1 then stays off
  s->ncu = (uint32_t)(ncu > 0 ? ncu : 0);
  // a test hook: phase 1's waits run out at once with LLMK_TEST_XS_SPIN=0
  const char* spin = getenv("LLMK_TEST_XS_SPIN");
  s->xs_spin = spin ? (uint32_t)strtoul(spin, nullptr, 10) : XS_SPIN;
  s->mem = mem;
  s->mem_bytes = L.total;
  s->ws = ws_carve((char*)mem, L, max_vocab, slots);
  *out = s;
  g_last_error.clear();
  return LLMK_OK;
}

extern "C" void llmk_sampler_destroy(llmk_sampler* s) {
  if (!s) return;
  (void)hipSetDevice(s->device);
  (void)hipDeviceSynchronize();
  (void)hipFree(s->mem);
  if (s->stage) (void)hipFree(s->stage);
  delete s;
}

extern "C" int llmk_sampler_status(llmk_sampler* s, void* stream,
                                   uint32_t* status) {
  if (!s || !status) return fail(LLMK_ERR_INVALID_ARGUMENT, "NULL argument");
  HIPCHK(hipSetDevice(s->device));
  hipStream_t st = (hipStream_t)stream;
  uint32_t v = 0;
  HIPCHK(hipMemcpyAsync(&v, s->ws.status, 4, hipMemcpyDeviceToHost, st));
  HIPCHK(hipStreamSynchronize(st));
  const uint32_t zero = 0;
  HIPCHK(hipMemcpyAsync(s->ws.status, &zero, 4, hipMemcpyHostToDevice, st));
  HIPCHK(hipStreamSynchronize(st));
  *status = v;
  return LLMK_OK;
}

// x rounded to nearest even into f32 (fmt 0), bf16 (1) or f16 (2), as a
// float: the scalar operand candle makes of an f64 for a tensor of that
// dtype (T::from_f64).  Subnormal results keep the format's fixed quantum;
// past the largest finite value the result is infinite.
static float dtype_round(double x, int fmt) {
  if (fmt == 0) return (float)x;
  if (x == 0.0 || !(x == x) || x - x != 0.0) return (float)x;
  const int p = fmt == 1 ? 8 : 11, emin = fmt == 1 ? -126 : -14, emax = fmt == 1 ? 127 : 15;
  int e = 0;
  (void)std::frexp(x, &e);  // x = f 2^e, 1/2 <= |f| < 1: the leading bit is 2^(e-1)
  const int lead = e - 1 < emin ? emin : e - 1;
  const double quantum = std::ldexp(1.0, lead - p + 1);
  const double r = std::nearbyint(x / quantum) * quantum;  // x / quantum is exact
  const double maxf = std::ldexp(2.0 - std::ldexp(1.0, 1 - p), emax);
  if (std::fabs(r) > maxf) return r > 0 ? __builtin_huge_valf() : -__builtin_huge_valf();
  return (float)r;
}

// One sampling launch on workspace ws, sized for batches up to max_batch rows
// of up to max_vocab logits with `pool` workgroup entries, on the current
// device.
// Phase 1 runs when it can pay for its launch (about 4 us): the call has
// top-k rows (only they are deferred) and at least XS_MIN_BATCH rows (at a
// few thousandths of rows failing the band check, fewer rows rarely have one).
constexpr uint32_t XS_MIN_BATCH = 16;
static int sample_batch_run(const Ws& ws, uint32_t max_batch, uint32_t max_vocab, uint32_t pool,
                            const llmk_sample_batch_args* in, void* stream, u4v* cut,
                            uint32_t tp_clamp, uint32_t epoch, uint32_t ncu,
                            uint32_t xs_spin = XS_SPIN) {
  if (!in) return fail(LLMK_ERR_INVALID_ARGUMENT, "args is NULL");
  if (in->vocab == 0) return fail(LLMK_ERR_EMPTY_LOGITS, "Empty logits passed to sampler");
  if (in->batch == 0) return fail(LLMK_ERR_INVALID_ARGUMENT, "batch is 0");
  if (!in->logits || !in->out_tokens || !in->uniforms)
    return fail(LLMK_ERR_INVALID_ARGUMENT, "logits, uniforms and out_tokens are required");
  if (in->dtype != LLMK_F32 && in->dtype != LLMK_BF16 && in->dtype != LLMK_F16)
    return fail(LLMK_ERR_INVALID_ARGUMENT, "dtype must be LLMK_F32, LLMK_BF16 or LLMK_F16");
  if (in->batch > max_batch || in->vocab > max_vocab)
    return fail(LLMK_ERR_CAPACITY, "batch or vocab above the sampler's maxima");
  if (in->row_stride < in->vocab)
    return fail(LLMK_ERR_INVALID_ARGUMENT, "row_stride < vocab");
  if ((in->hist_offsets == nullptr) != (in->hist_tokens == nullptr))
    return fail(LLMK_ERR_INVALID_ARGUMENT, "hist_offsets and hist_tokens go together");
  if (in->hist_lengths && !in->hist_offsets)
    return fail(LLMK_ERR_INVALID_ARGUMENT, "hist_lengths needs hist_offsets and hist_tokens");
  if (in->hist_counts && !in->hist_offsets)
    return fail(LLMK_ERR_INVALID_ARGUMENT, "hist_counts needs hist_offsets and hist_tokens");
  if (in->allow_mask && in->mask_words_per_row < (in->vocab + 31) / 32)
    return fail(LLMK_ERR_INVALID_ARGUMENT, "mask_words_per_row < ceil(vocab/32)");
  if (in->out_cap && !in->out_ids && !in->out_probs)
    return fail(LLMK_ERR_INVALID_ARGUMENT, "out_cap without out_ids/out_probs");
  if (!(in->softcap >= 0.0f) || !(in->softcap < __builtin_huge_valf()))
    return fail(LLMK_ERR_INVALID_ARGUMENT, "softcap must be finite and >= 0 (0 = off)");
  const size_t esz = in->dtype == LLMK_F32 ? 4 : 2;
  const size_t align = 16;  // the tiles' 16-byte loads
  if (((uintptr_t)in->logits % align) != 0 || ((in->row_stride * esz) % align) != 0)
    return fail(LLMK_ERR_ALIGNMENT, "logit rows must be 16-byte aligned");

  Args a;
  a.logits = in->logits;
  a.dtype = in->dtype;
  a.sc_m1 = a.sc_cap = 0.0f;
  if (in->softcap > 0.0f) {
    // candle's scalar operands: 1/cap in f64, then the tensor's dtype
    const int fmt = in->dtype == LLMK_F32 ? 0 : (in->dtype == LLMK_BF16 ? 1 : 2);
    a.sc_m1 = dtype_round(1.0 / (double)in->softcap, fmt);
    a.sc_cap = dtype_round((double)in->softcap, fmt);
  }
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
  a.hlen = in->hist_lengths;
  a.hcnt = in->hist_counts;
  a.mask = in->allow_mask;
  a.mask_words = in->mask_words_per_row;
  a.u = in->uniforms;
  a.out_tok = in->out_tokens;
  a.out_ids = in->out_ids;
  a.out_cnt = in->out_count;
  a.out_probs = in->out_probs;
  a.out_cap = in->out_cap;
  a.cut = cut;
  a.tp_clamp = tp_clamp;
  a.phase = 0;
  // phase 1's grid (jobs x windows) fits the GPU at one workgroup a CU, so
  // a window's wait for the sums before it always ends
  const uint32_t nwin = xs_maxw(in->vocab);
  const bool phase1 = in->top_k != nullptr && in->batch >= XS_MIN_BATCH;
  // (jobs x windows within the device's CUs: every workgroup resident)
  a.xs_cap = !phase1 ? 0u : (ncu / nwin < XS_JOBS ? ncu / nwin : XS_JOBS);
  a.xs_lds = 0;
  a.epoch = epoch;
  a.xs_spin = xs_spin;
  a.ntiles = (a.V + TILE - 1) / TILE;
  a.nchunks = (a.ntiles + CHUNK_TILES - 1) / CHUNK_TILES;
  // Segments per row: enough workgroups to cover the 256 CUs, whole 16-tile
  // chunks per segment, at most MAX_SEG segments.
  uint32_t G = (256 + a.B - 1) / a.B;
  if (G > a.nchunks) G = a.nchunks;
  if (G > MAX_SEG) G = MAX_SEG;
  if (G < 1) G = 1;
  while (G > 1 && (uint64_t)a.B * G > pool) --G;
  const uint32_t cps = (a.nchunks + G - 1) / G;  // chunks per segment
  a.tps = cps * CHUNK_TILES;
  a.G = (a.nchunks + cps - 1) / cps;
  a.xcd_map = (a.G > 1 && (a.B % 8) == 0) ? 1u : 0u;

  hipStream_t st = (hipStream_t)stream;
  size_t words = stream_lds_words(a.tps);
  if (finalize_lds_words() > words) words = finalize_lds_words();
  // a single-segment row keeps its partials and first candidates past both
  words = (words + 3) & ~(size_t)3;
  a.lds_part = (uint32_t)words;
  a.lds_cand = a.lds_part + 2 * MAX_SLOTS;
  if (a.G == 1) words = a.lds_cand + 2 * LCAP;
  if (slow_lds_words(a.V) > words) words = slow_lds_words(a.V);
  const size_t lds = 4 * words;
  if (lds > LDS_DYN_MAX)
    return fail(LLMK_ERR_CAPACITY, "vocabulary too large for one workgroup's LDS tables");
  const bool sc = in->softcap > 0.0f;
  auto launch = [&](const Args& x, dim3 grid, size_t bytes) {
    const dim3 block(NT);
    const int v = (x.dtype == LLMK_F32 ? 0 : x.dtype == LLMK_BF16 ? 2 : 4) + (sc ? 1 : 0);
    if (x.phase == 0) {
      switch (v) {
        case 0: hipLaunchKernelGGL(stream_kernel<LLMK_F32>, grid, block, bytes, st, x, ws); break;
        case 1: hipLaunchKernelGGL(stream_kernel<LLMK_F32 | SOFTCAP>, grid, block, bytes, st, x, ws); break;
        case 2: hipLaunchKernelGGL(stream_kernel<LLMK_BF16>, grid, block, bytes, st, x, ws); break;
        case 3: hipLaunchKernelGGL(stream_kernel<LLMK_BF16 | SOFTCAP>, grid, block, bytes, st, x, ws); break;
        case 4: hipLaunchKernelGGL(stream_kernel<LLMK_F16>, grid, block, bytes, st, x, ws); break;
        default: hipLaunchKernelGGL(stream_kernel<LLMK_F16 | SOFTCAP>, grid, block, bytes, st, x, ws);
      }
    } else {
      switch (v) {
        case 0: hipLaunchKernelGGL(xs_kernel<LLMK_F32>, grid, block, bytes, st, x, ws); break;
        case 1: hipLaunchKernelGGL(xs_kernel<LLMK_F32 | SOFTCAP>, grid, block, bytes, st, x, ws); break;
        case 2: hipLaunchKernelGGL(xs_kernel<LLMK_BF16>, grid, block, bytes, st, x, ws); break;
        case 3: hipLaunchKernelGGL(xs_kernel<LLMK_BF16 | SOFTCAP>, grid, block, bytes, st, x, ws); break;
        case 4: hipLaunchKernelGGL(xs_kernel<LLMK_F16>, grid, block, bytes, st, x, ws); break;
        default: hipLaunchKernelGGL(xs_kernel<LLMK_F16 | SOFTCAP>, grid, block, bytes, st, x, ws);
      }
    }
  };
  launch(a, dim3(a.B * a.G), lds);
  HIPCHK(hipGetLastError());
  // phase 1: the S of the rows whose band check failed (most calls have
  // none: each workgroup then reads the job count and ends)
  if (a.xs_cap > 0) {
    Args a1 = a;
    a1.phase = 1;
    // (a window's history tables and packing space; window 0's copy of its
    // records, terms and runs takes the tables' place afterwards)
    const size_t own = 128 + (size_t)NW * (TILE + XS_RUNW);
    const size_t hist = hist_lds_words(XS_W / 32) + NW * XS_CW;
    const size_t lds1 = 4 * (256 + (hist > own ? hist : own));
    a1.xs_lds = (uint32_t)((lds > lds1 ? lds : lds1) / 4);
    launch(a1, dim3(a.xs_cap * nwin), 4 * (size_t)a1.xs_lds);
    HIPCHK(hipGetLastError());
  }
  return LLMK_OK;
}

// Rows at any element offset (sampler.rs:25-29 samples any &[f32], which
// candle.rs:2007-2009 narrows from the lm_head output at any offset): copied
// element by element, each read at its own alignment, into rows of stride
// round_up(V, 8) that start 16-byte aligned, which the sampling kernel reads.
__global__ __launch_bounds__(256) void realign_kernel(const void* src, uint64_t src_stride,
                                                      void* dst, uint64_t dst_stride, uint32_t V,
                                                      uint32_t esz) {
  const uint32_t b = blockIdx.y;
  for (uint32_t k = 0; k < 4; ++k) {
    const uint32_t e = blockIdx.x * 1024u + 256u * k + threadIdx.x;
    if (e >= V) break;
    if (esz == 4)
      G((float*)dst)[(uint64_t)b * dst_stride + e] =
          G((const float*)src)[(uint64_t)b * src_stride + e];
    else
      G((uint16_t*)dst)[(uint64_t)b * dst_stride + e] =
          G((const uint16_t*)src)[(uint64_t)b * src_stride + e];
  }
}

static int sample_batch_impl(llmk_sampler* s, const llmk_sample_batch_args* in,
                             void* stream, u4v* cut, uint32_t tp_clamp) {
  if (!s) return fail(LLMK_ERR_INVALID_ARGUMENT, "sampler is NULL");
  HIPCHK(hipSetDevice(s->device));
  const uint32_t pool = s->max_batch > MAX_WGS ? s->max_batch : MAX_WGS;
  const size_t esz = in && in->dtype == LLMK_F32 ? 4 : 2;
  const bool valid = in && in->logits && in->batch > 0 && in->vocab > 0 &&
                     in->batch <= s->max_batch && in->vocab <= s->max_vocab &&
                     in->row_stride >= in->vocab &&
                     (in->dtype == LLMK_F32 || in->dtype == LLMK_BF16 || in->dtype == LLMK_F16);
  if (valid &&
      (((uintptr_t)in->logits % 16) != 0 || ((in->row_stride * esz) % 16) != 0)) {
    // rows at any offset: their aligned copies (the staging rows grow on
    // demand; the call then allocates, once)
    const uint64_t dstride = ((uint64_t)in->vocab + 7) / 8 * 8;
    const size_t need = (size_t)in->batch * dstride * esz;
    if (need > s->stage_bytes) {
      HIPCHK(hipDeviceSynchronize());  // an earlier call may still read the old rows
      if (s->stage) HIPCHK(hipFree(s->stage));
      s->stage = nullptr;
      s->stage_bytes = 0;
      HIPCHK(hipMalloc(&s->stage, need));
      s->stage_bytes = need;
    }
    hipLaunchKernelGGL(realign_kernel, dim3((in->vocab + 1023) / 1024, in->batch), dim3(256), 0,
                       (hipStream_t)stream, in->logits, in->row_stride, s->stage, dstride,
                       in->vocab, (uint32_t)esz);
    HIPCHK(hipGetLastError());
    llmk_sample_batch_args al = *in;
    al.logits = s->stage;
    al.row_stride = dstride;
    const int rc = sample_batch_run(s->ws, s->max_batch, s->max_vocab, pool, &al, stream, cut,
                                    tp_clamp, s->epoch, s->ncu, s->xs_spin);
    if (rc == LLMK_OK) ++s->epoch;  // the parity advances with the launches only
    return rc;
  }
  const int rc = sample_batch_run(s->ws, s->max_batch, s->max_vocab, pool, in, stream, cut,
                                  tp_clamp, s->epoch, s->ncu, s->xs_spin);
  if (rc == LLMK_OK) ++s->epoch;
  return rc;
}

extern "C" int llmk_sample_batch(llmk_sampler* s, const llmk_sample_batch_args* in,
                                 void* stream) {
  return sample_batch_impl(s, in, stream, nullptr, 0u);
}

// ---- llmk_sample_batch_static: the sampling call with no allocation ------
// Limits of the static workspace: batches up to 256 rows of up to 2^18
// logits, 512 workgroup entries (B x G stays below 256 + B <= 512 for every
// B <= 256, so the launch shape is that of a handle) and 8 slow-path slots
// (rows b, b + 8, ... share one; a row waits for its slot's holder).
constexpr uint32_t STATIC_MAX_BATCH = 256;
constexpr uint32_t STATIC_MAX_VOCAB = 1u << 18;
constexpr uint32_t STATIC_POOL = 512;
constexpr uint32_t STATIC_SLOTS = 8;
constexpr WsLayout STATIC_LAYOUT =
    ws_layout(STATIC_MAX_BATCH, STATIC_MAX_VOCAB, STATIC_POOL, STATIC_SLOTS);
static_assert(STATIC_LAYOUT.total <= (160ull << 20), "static workspace above 160 MiB");

// One copy per GPU, held until the process ends.  Host code must not use
// this name as an address: it is a host-side stand-in for the symbol; the
// device address comes from hipGetSymbolAddress.
static __device__ __align__(256) uint8_t scratch[STATIC_LAYOUT.total];

constexpr int STATIC_MAX_DEVICES = 64;
static std::mutex g_static_mu;
static char* g_static_ptr[STATIC_MAX_DEVICES];  // device address of scratch, per device
static uint32_t g_static_ncu[STATIC_MAX_DEVICES];  // compute units, per device

// Clears what every call must find at zero: the rows' arrival counters, the
// slow-path slot locks and the status word (a fill kernel, so the call can
// be captured in a HIP graph).
__global__ __launch_bounds__(256) void static_clear_kernel(uint32_t* arrive, uint32_t n_arrive,
                                                           uint32_t* lock, uint32_t n_lock,
                                                           uint32_t* status, uint32_t* xs_ctl) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i < n_arrive) arrive[i] = 0;
  if (i < n_lock) lock[i] = 0;
  if (i == 0) status[0] = 0;
  if (i < XS_CTL_WORDS) xs_ctl[i] = 0;
}

// Device address of this device's scratch array, looked up (and the
// kernels' LDS limits set) on the first call on each device.
static int static_scratch(int dev, char** out, uint32_t* ncu) {
  if (dev < 0 || dev >= STATIC_MAX_DEVICES)
    return fail(LLMK_ERR_UNSUPPORTED, "device ordinal above 63");
  std::lock_guard<std::mutex> g(g_static_mu);
  if (!g_static_ptr[dev]) {
    const int rc = set_kernel_attributes();
    if (rc != LLMK_OK) return rc;
    void* ptr = nullptr;
    HIPCHK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    if (!ptr) return fail(LLMK_ERR_HIP, "hipGetSymbolAddress(scratch) returned NULL");
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) n = 0;
    g_static_ncu[dev] = (uint32_t)(n > 0 ? n : 0);
    g_static_ptr[dev] = (char*)ptr;
  }
  *out = g_static_ptr[dev];
  *ncu = g_static_ncu[dev];
  return LLMK_OK;
}

extern "C" int llmk_sample_batch_static(const llmk_sample_batch_args* in, uint32_t* status,
                                        void* stream) {
  if (!in) return fail(LLMK_ERR_INVALID_ARGUMENT, "args is NULL");
  if (in->batch > STATIC_MAX_BATCH || in->vocab > STATIC_MAX_VOCAB)
    return fail(LLMK_ERR_CAPACITY,
                "llmk_sample_batch_static serves batch <= 256 and vocab <= 262144 (got batch " +
                    std::to_string(in->batch) + ", vocab " + std::to_string(in->vocab) +
                    "); use a handle from llmk_sampler_create");
  int dev = 0;
  HIPCHK(hipGetDevice(&dev));
  char* base = nullptr;
  uint32_t ncu = 0;
  const int rc = static_scratch(dev, &base, &ncu);
  if (rc != LLMK_OK) return rc;
  Ws ws = ws_carve(base, STATIC_LAYOUT, STATIC_MAX_VOCAB, STATIC_SLOTS);
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(static_clear_kernel, dim3((STATIC_MAX_BATCH + 255) / 256), dim3(256), 0, st,
                     ws.row_arrive, STATIC_MAX_BATCH, ws.slow_lock, STATIC_SLOTS, ws.status,
                     ws.xs_ctl);
  HIPCHK(hipGetLastError());
  if (status) ws.status = status;
  // the clear kernel zeroed both job counts: every call can use parity 0
  return sample_batch_run(ws, STATIC_MAX_BATCH, STATIC_MAX_VOCAB, STATIC_POOL, in, stream,
                          nullptr, 0u, 0u, ncu);
}

// Checks shared by the mask forms: in-place f32 rows.
static int check_mask_rows(llmk_sampler* s, const float* logits, uint32_t vocab,
                           uint64_t row_stride, const void* param) {
  if (!s) return fail(LLMK_ERR_INVALID_ARGUMENT, "sampler is NULL");
  if (!logits || !param) return fail(LLMK_ERR_INVALID_ARGUMENT, "logits and the parameter array are required");
  if (row_stride < vocab) return fail(LLMK_ERR_INVALID_ARGUMENT, "row_stride < vocab");
  if (((uintptr_t)logits % 4) != 0) return fail(LLMK_ERR_ALIGNMENT, "logits must be 4-byte aligned");
  if (vocab > MAX_TILES * TILE) return fail(LLMK_ERR_CAPACITY, "vocab above 2^20");
  return LLMK_OK;
}

extern "C" int llmk_apply_top_k(llmk_sampler* s, float* logits, uint32_t batch, uint32_t vocab,
                                uint64_t row_stride, const int32_t* top_k, void* stream) {
  const int rc = check_mask_rows(s, logits, vocab, row_stride, top_k);
  if (rc != LLMK_OK) return rc;
  if (batch == 0 || vocab == 0) return LLMK_OK;  // nothing to mask (sampler.rs:161)
  HIPCHK(hipSetDevice(s->device));
  hipLaunchKernelGGL(topk_mask_kernel, dim3(batch), dim3(NT), 4 * MK_LDS_WORDS,
                     (hipStream_t)stream, logits, vocab, row_stride, top_k);
  HIPCHK(hipGetLastError());
  return LLMK_OK;
}

extern "C" int llmk_apply_top_p(llmk_sampler* s, float* logits, uint32_t batch, uint32_t vocab,
                                uint64_t row_stride, const float* top_p, void* stream) {
  const int rc = check_mask_rows(s, logits, vocab, row_stride, top_p);
  if (rc != LLMK_OK) return rc;
  if (batch == 0 || vocab == 0) return LLMK_OK;
  if (batch > s->max_batch || vocab > s->max_vocab)
    return fail(LLMK_ERR_CAPACITY, "batch or vocab above the sampler's maxima");
  // the cut: the sampling kernel at temperature 1 with top_p alone
  llmk_sample_batch_args in;
  memset(&in, 0, sizeof(in));
  in.logits = logits;
  in.dtype = LLMK_F32;
  in.batch = batch;
  in.vocab = vocab;
  in.row_stride = row_stride;
  in.top_p = top_p;
  in.uniforms = s->ws.zu;
  in.out_tokens = s->ws.mtok;
  const int rc2 = sample_batch_impl(s, &in, stream, s->ws.cut, 1u);
  if (rc2 != LLMK_OK) return rc2;
  // then the mask, in segments of whole 4096-element blocks, ~2048 workgroups
  const uint32_t blocks = (vocab + 4 * NT - 1) / (4 * NT);
  uint32_t want = (2048 + batch - 1) / batch;
  if (want > blocks) want = blocks;
  const uint32_t seg = (blocks + want - 1) / want * (4 * NT);
  const uint32_t nseg = (vocab + seg - 1) / seg;
  hipLaunchKernelGGL(topp_mask_kernel, dim3(batch * nseg), dim3(NT), 0, (hipStream_t)stream,
                     logits, vocab, row_stride, top_p, (const u4v*)s->ws.cut, s->ws.mtok,
                     nseg, seg);
  HIPCHK(hipGetLastError());
  return LLMK_OK;
}

extern "C" int llmk_apply_logit_bias(llmk_sampler* s, float* logits, uint32_t batch,
                                     uint32_t vocab, uint64_t row_stride,
                                     const uint32_t* bias_offsets, const uint32_t* bias_tokens,
                                     const float* bias_values, void* stream) {
  const int rc = check_mask_rows(s, logits, vocab, row_stride, bias_offsets);
  if (rc != LLMK_OK) return rc;
  if (!bias_tokens || !bias_values)
    return fail(LLMK_ERR_INVALID_ARGUMENT, "bias_tokens and bias_values are required");
  if (batch == 0 || vocab == 0) return LLMK_OK;
  HIPCHK(hipSetDevice(s->device));
  hipLaunchKernelGGL(logit_bias_kernel, dim3((batch + NW - 1) / NW), dim3(NT), 0,
                     (hipStream_t)stream, logits, batch, vocab, row_stride, bias_offsets,
                     bias_tokens, bias_values);
  HIPCHK(hipGetLastError());
  return LLMK_OK;
}

extern "C" int llmk_verify_batch(llmk_sampler* s, uint32_t batch, uint32_t vocab,
                                 const uint32_t* ids, const float* probs, uint32_t list_cap,
                                 const uint32_t* counts, const uint32_t* draft_tokens,
                                 const float* draft_probs, uint64_t draft_stride,
                                 const float* u_accept, const float* u_resample,
                                 uint32_t* out_tokens, uint32_t* out_accepted, void* stream) {
  if (!s) return fail(LLMK_ERR_INVALID_ARGUMENT, "sampler is NULL");
  if (vocab == 0) return fail(LLMK_ERR_EMPTY_LOGITS, "Empty logits passed to sampler");
  if (!ids || !probs || !counts || !draft_tokens || !draft_probs || !u_accept || !u_resample ||
      !out_tokens || !out_accepted)
    return fail(LLMK_ERR_INVALID_ARGUMENT, "every array of llmk_verify_batch is required");
  if (list_cap == 0) return fail(LLMK_ERR_INVALID_ARGUMENT, "list_cap is 0");
  if (draft_stride < vocab) return fail(LLMK_ERR_INVALID_ARGUMENT, "draft_stride < vocab");
  if (batch == 0) return LLMK_OK;
  HIPCHK(hipSetDevice(s->device));
  VerifyArgs v{batch, vocab, list_cap, ids, probs, counts, draft_tokens, draft_probs,
               draft_stride, u_accept, u_resample, out_tokens, out_accepted};
  hipLaunchKernelGGL(verify_kernel, dim3(batch), dim3(WAVE), 0, (hipStream_t)stream, v,
                     s->ws.status);
  HIPCHK(hipGetLastError());
  return LLMK_OK;
}

extern "C" int llmk_history_count_append(llmk_sampler* s, uint32_t batch,
                                         const uint32_t* hist_offsets, uint32_t* hist_lengths,
                                         uint32_t* hist_tokens, uint32_t* hist_counts,
                                         uint32_t capacity, const uint32_t* tokens,
                                         void* stream) {
  if (!s) return fail(LLMK_ERR_INVALID_ARGUMENT, "sampler is NULL");
  if (!hist_offsets || !hist_lengths || !hist_tokens || !hist_counts || !tokens)
    return fail(LLMK_ERR_INVALID_ARGUMENT, "history arrays, counts and tokens are required");
  if (batch == 0) return LLMK_OK;
  HIPCHK(hipSetDevice(s->device));
  hipLaunchKernelGGL(history_count_append_kernel, dim3(batch), dim3(HCA_T), 0,
                     (hipStream_t)stream, hist_offsets, hist_lengths, hist_tokens, hist_counts,
                     capacity, tokens, s->ws.status);
  HIPCHK(hipGetLastError());
  return LLMK_OK;
}

extern "C" int llmk_history_append(llmk_sampler* s, uint32_t batch, const uint32_t* hist_offsets,
                                   uint32_t* hist_lengths, uint32_t* hist_tokens,
                                   uint32_t capacity, const uint32_t* tokens, void* stream) {
  if (!s) return fail(LLMK_ERR_INVALID_ARGUMENT, "sampler is NULL");
  if (!hist_offsets || !hist_lengths || !hist_tokens || !tokens)
    return fail(LLMK_ERR_INVALID_ARGUMENT, "history arrays and tokens are required");
  if (batch == 0) return LLMK_OK;
  HIPCHK(hipSetDevice(s->device));
  hipLaunchKernelGGL(history_append_kernel, dim3((batch + 255) / 256), dim3(256), 0,
                     (hipStream_t)stream, batch, hist_offsets, hist_lengths, hist_tokens,
                     capacity, tokens, s->ws.status);
  HIPCHK(hipGetLastError());
  return LLMK_OK;
}
