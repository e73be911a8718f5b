// Router: the gate GEMV (logits = x . Wr) and softmax + top-k.
//
// The reference runs the gate linear as an MLX matmul and the top-k in moe_probs, one 32-lane warp a row doing k
// rounds of shuffle argmax (route_cuda.py:193-254). Here:
//   * k_router_gemv gives each router row a workgroup (256 threads, 8 weights a thread a step, x read straight
//     into registers), and emits the prepared activation rows the expert kernels read (lmoe_common.h), so no
//     later kernel rearranges x again;
//   * k_router_topk takes k rounds of a wavefront argmax, one wavefront a token, its max and min-index reductions
//     on DPP and gfx950's permlane swaps rather than LDS shuffles.
// Selection is on the fp32 logits, larger first, ties to the lower expert index; scores are the softmax
// probabilities of the picked experts (max-subtracted, fp32), renormalised when asked.
#include "lmoe_common.h"

#include <cstdlib>
#include <type_traits>

namespace lmoe {

constexpr int kMaxNpl = 16;  // logits a lane: E <= 64 * 16

// Four tokens a workgroup, one wavefront each (k_router_topk's body).
template <int NPL>
__device__ __forceinline__ void topk_rows(int block, const void *logits, int ldt, int ld_stride, int T, int E,
                                          int k, int norm, uint32_t *ids, float *scores, const float *gate, int m) {
  __shared__ __attribute__((aligned(16))) uint32_t scr[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = block * 4 + wave;
  if (t >= T) return;
  const size_t base = size_t(t) * ld_stride;
  float v[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int i = lane + 64 * j;
    v[j] = i < E ? load_elt(logits, base + i, ldt) : -INFINITY;
  }
  uint32_t id;
  float sc;
  topk_wave<NPL>(v, E, k, norm, scr[wave], &id, &sc);
  const int ks = k + m;
  if (lane < k) {
    ids[size_t(t) * ks + lane] = id;
    scores[size_t(t) * ks + lane] = sc;
  } else if (lane < ks) {
    ids[size_t(t) * ks + lane] = uint32_t(E + lane - k);
    scores[size_t(t) * ks + lane] = sigmoidf_(gate[t]);
  }
}

// Four tokens a workgroup, one wavefront each.
// m > 0: each token's ids / scores rows hold k + m entries, the last m the folded shared expert's slices
// (E + j, sigmoid(gate[t])).
template <int NPL>
__global__ void __launch_bounds__(256) k_router_topk(const void *logits, int ldt, int ld_stride, int T, int E,
                                                     int k, int norm, uint32_t *ids, float *scores,
                                                     const float *gate = nullptr, int m = 0) {
  topk_rows<NPL>(blockIdx.x, logits, ldt, ld_stride, T, E, k, norm, ids, scores, gate, m);
}

// The prefill's top-k and x's conversion to f16 in the GEMM K order (the two steps before the grouping that do not
// depend on each other, when the logits are given) as one launch: workgroups [0, nb_topk) rank four tokens each,
// the rest convert 2,048 elements each. One kernel boundary fewer, and the two overlap on the chip.
template <int NPL>
__global__ void __launch_bounds__(256) k_topk_and_f16(const void *logits, int ldt, int T, int E, int k, int norm,
                                                      uint32_t *ids, float *scores, int nb_topk, const void *x,
                                                      int xdt, long long n, _Float16 *xh) {
  if (int(blockIdx.x) < nb_topk)
    topk_rows<NPL>(blockIdx.x, logits, ldt, E, T, E, k, norm, ids, scores, nullptr, 0);
  else
    to_f16_kperm(blockIdx.x - nb_topk, x, xdt, n, xh);
}

constexpr int kRouterMaxT = 16;
constexpr int kRouterMaxNi = 4;  // 8-weight items a thread: H <= 8192

// One workgroup a router row (row E: the shared-expert gate, when wsg is given). Thread i holds the row's 8-weight
// items i, i + 256, ... (NI of them, 16-byte loads issued first) and, token by token, the matching 8 values of x
// straight from memory (no staging); a wavefront sum and a fixed-order sum of the four wavefronts' partials give
// the logit. Workgroups past the rows write the prepared activation units for block type TQ (when xprep is given),
// four units a workgroup, one a wavefront through its own LDS. WDT: the weights' element type.
template <int WDT, int TQ, int NI, bool TL = false>
__global__ void __launch_bounds__(256)
    k_router_gemv(const void *x, int xdt, const void *wr, const void *wsg, int T, int H, int E, float *logits,
                  uint32_t *xprep, unsigned long long *tl) {
  constexpr int WQ = WDT == LMOE_F32 ? 2 : 1;  // 16-byte chunks an item of weights
  __shared__ float part[4][kRouterMaxT];
  __shared__ float xu[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rows = E + (wsg != nullptr ? 1 : 0);
  const int row = blockIdx.x;
  const int nit = H / 8;
  tl_stamp<TL>(tl, 0);
  if (row >= rows) {  // a prepared-activation workgroup: one unit a wavefront, wavefront-private LDS
    const int P = H / 64;
    const int u = (row - rows) * 4 + wave;
    if (u >= T * P) return;
    const int t = u / P, p = u - t * P;
    xu[wave][lane] = load_elt(x, size_t(t) * H + 64 * p + lane, xdt);
    __builtin_amdgcn_wave_barrier();
    if (lane < XS) xprep[size_t(u) * XS + lane] = prep_dword<TQ>([&](int i) { return xu[wave][i]; }, 0, lane);
    tl_stamp<TL>(tl, 4);
    return;
  }
  const u32x4 *w4 = reinterpret_cast<const u32x4 *>(
      row < E ? static_cast<const char *>(wr) + size_t(row) * H * (WDT == LMOE_F32 ? 4 : 2)
              : static_cast<const char *>(wsg));
  u32x4 wq[NI][2];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int it = min(int(threadIdx.x) + 256 * i, nit - 1);  // not predicated: past the row, the last item again
#pragma unroll
    for (int q = 0; q < WQ; ++q) wq[i][q] = __builtin_nontemporal_load(w4 + it * WQ + q);
  }
  // token t's x items (the first token's go out with the weights, before anything waits on them)
  const int xq = xdt == LMOE_F32 ? 2 : 1;  // 16-byte chunks an item of x
  u32x4 xc[NI][2];
  auto load_x = [&](int t) {
    const u32x4 *x4 = reinterpret_cast<const u32x4 *>(static_cast<const char *>(x) +
                                                      size_t(t) * H * (xdt == LMOE_F32 ? 4 : 2));
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int it = min(int(threadIdx.x) + 256 * i, nit - 1);
      xc[i][0] = x4[it * xq];
      xc[i][1] = x4[it * xq + xq - 1];
    }
  };
  load_x(0);
  asm volatile("" ::: "memory");  // keeps them here, not sunk into the dot loop's per-lane branch behind the weights
  float wv[NI][8];
#pragma unroll
  for (int i = 0; i < NI; ++i) unpack8(wq[i][0], wq[i][WQ - 1], WDT, wv[i]);
  if constexpr (TL) {
    asm volatile("" ::"v"(wv[0][0]), "v"(wv[NI - 1][7]));
    tl_stamp<TL>(tl, 3);
  }
  for (int t = 0; t < T; ++t) {
    if (t > 0) load_x(t);
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      if (int(threadIdx.x) + 256 * i >= nit) continue;
      float xv[8];
      unpack8(xc[i][0], xc[i][1], xdt, xv);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc = fmaf(xv[e], wv[i][e], acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) part[wave][t] = acc;
  }
  __syncthreads();
  if (threadIdx.x < T)
    logits[size_t(threadIdx.x) * rows + row] =
        ((part[0][threadIdx.x] + part[1][threadIdx.x]) + part[2][threadIdx.x]) + part[3][threadIdx.x];
  tl_stamp<TL>(tl, 4);
}

// Prepared activation rows on their own: one workgroup a row, one thread a unit dword.
template <int TQ>
__global__ void __launch_bounds__(256) k_prep_x(const void *x, int xdt, int H, uint32_t *xprep) {
  const int P = H / 64;
  const size_t r = blockIdx.y;
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= P * XS) return;
  const int p = idx / XS, dw = idx - p * XS;
  xprep[r * P * XS + idx] = prep_dword<TQ>([&](int i) { return load_elt(x, r * H + i, xdt); }, p, dw);
}

template <int WDT, int TQ>
static void launch_router_q(dim3 grid, dim3 block, hipStream_t st, const void *x, int xdt, const void *wr,
                            const void *wsg, int T, int H, int E, float *logits, uint32_t *xprep) {
  const int ni = (H / 8 + 255) / 256;
  unsigned long long *tl = timeline_next(LMOE_TL_ROUTER, int(grid.x * grid.y));
  auto go = [&](auto nic) {
    constexpr int NI = decltype(nic)::value;
    if (tl)
      launch(k_router_gemv<WDT, TQ, NI, true>, grid, block, 0, st, x, xdt, wr, wsg, T, H, E, logits, xprep, tl);
    else
      launch(k_router_gemv<WDT, TQ, NI>, grid, block, 0, st, x, xdt, wr, wsg, T, H, E, logits, xprep, tl);
  };
  if (ni <= 1)
    go(std::integral_constant<int, 1>());
  else if (ni <= 2)
    go(std::integral_constant<int, 2>());
  else
    go(std::integral_constant<int, 4>());
}

template <int WDT>
static void launch_router(int qt, dim3 grid, dim3 block, hipStream_t st, const void *x, int xdt, const void *wr,
                          const void *wsg, int T, int H, int E, float *logits, uint32_t *xprep) {
  if (qt == LMOE_Q4_K)
    launch_router_q<WDT, LMOE_Q4_K>(grid, block, st, x, xdt, wr, wsg, T, H, E, logits, xprep);
  else
    launch_router_q<WDT, LMOE_Q4_0>(grid, block, st, x, xdt, wr, wsg, T, H, E, logits, xprep);
}


// ---- router GEMV and top-k in one launch ------------------------------------------------------------------------
//
// Workgroup g < NR computes router rows [8 g, 8 g + 8) (row E: the shared-expert gate) for every token, each row in
// exactly k_router_gemv's order (thread i holds items i, i + 256, ...; a wavefront tree; the four wavefronts' totals
// left to right), so the logits are bit-for-bit those of lmoe_router_gemv. It then counts itself in on a device
// counter (release); the workgroup that arrives last (acquire) ranks each token's logits, writes ids / scores, and
// resets the counter for the next launch. Nobody waits on anybody: with NR = ceil((E + 1) / 8) workgroups the
// counter sees ~17 arrivals for E 128 instead of a kernel boundary and a top-k in every gate/up wavefront.
// Workgroups past NR write the prepared activation rows, as in k_router_gemv.
// ks: slots a token in ids / scores (k, or k + m with a shared expert folded in as slots k..k+m-1: ids E.., weight
// sigmoid(gate logit)). sync: a device counter, zero before the first launch, left zero by every launch.
template <int WDT, int TQ, int NI, int kRankRows>
__global__ void __launch_bounds__(256)
    k_router_rank(const void *x, int xdt, const void *wr, const void *wsg, int T, int H, int E, int k, int norm,
                  int ks, float *logits, uint32_t *ids, float *scores, uint32_t *xprep, uint32_t *sync, int nr) {
  constexpr int WQ = WDT == LMOE_F32 ? 2 : 1;
  __shared__ float part[kRankRows][4];
  __shared__ float xu[4][64];
  __shared__ int last;
  __shared__ __attribute__((aligned(16))) RankScratch rs;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rows = E + (wsg != nullptr ? 1 : 0);
  const int nit = H / 8;
  if (int(blockIdx.x) >= nr) {  // a prepared-activation workgroup: one unit a wavefront
    const int P = H / 64;
    const int u = (blockIdx.x - nr) * 4 + wave;
    if (u >= T * P) return;
    const int t = u / P, p = u - t * P;
    xu[wave][lane] = load_elt(x, size_t(t) * H + 64 * p + lane, xdt);
    __builtin_amdgcn_wave_barrier();
    if (lane < XS) xprep[size_t(u) * XS + lane] = prep_dword<TQ>([&](int i) { return xu[wave][i]; }, 0, lane);
    return;
  }
  const int r0 = blockIdx.x * kRankRows;
  float wv[kRankRows][NI][8];
#pragma unroll
  for (int r = 0; r < kRankRows; ++r) {
    const int row = min(r0 + r, rows - 1);
    const u32x4 *w4 = reinterpret_cast<const u32x4 *>(
        row < E ? static_cast<const char *>(wr) + size_t(row) * H * (WDT == LMOE_F32 ? 4 : 2)
                : static_cast<const char *>(wsg));
    u32x4 wq[NI][2];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int it = min(tid + 256 * i, nit - 1);
#pragma unroll
      for (int q = 0; q < WQ; ++q) wq[i][q] = __builtin_nontemporal_load(w4 + it * WQ + q);
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) unpack8(wq[i][0], wq[i][WQ - 1], WDT, wv[r][i]);
  }
  const int xq = xdt == LMOE_F32 ? 2 : 1;
  for (int t = 0; t < T; ++t) {
    const u32x4 *x4 = reinterpret_cast<const u32x4 *>(static_cast<const char *>(x) +
                                                      size_t(t) * H * (xdt == LMOE_F32 ? 4 : 2));
    float xv[NI][8];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int it = min(tid + 256 * i, nit - 1);
      unpack8(x4[it * xq], x4[it * xq + xq - 1], xdt, xv[i]);
    }
#pragma unroll
    for (int r = 0; r < kRankRows; ++r) {
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        if (tid + 256 * i >= nit) continue;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc = fmaf(xv[i][e], wv[r][i][e], acc);
      }
      acc = wave_sum(acc);
      if (lane == 0) part[r][wave] = acc;
    }
    __syncthreads();
    if (tid < kRankRows && r0 + tid < rows)
      logits[size_t(t) * rows + r0 + tid] = ((part[tid][0] + part[tid][1]) + part[tid][2]) + part[tid][3];
    __syncthreads();
  }
  // count in; the last workgroup ranks
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(sync, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    last = prev == uint32_t(nr - 1);
  }
  __syncthreads();
  if (!last) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  if (tid == 0) __hip_atomic_store(sync, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (int t = 0; t < T; ++t) {
    for (int e = tid; e < rows; e += 256) rs.vals[e] = logits[size_t(t) * rows + e];
    __syncthreads();
    const float p = rank256(rs, E, k, norm, tid);
    if (tid < k) {
      ids[size_t(t) * ks + tid] = rs.pick[tid];
      scores[size_t(t) * ks + tid] = p;
    }
    if (tid >= k && tid < ks) {  // the folded shared expert's slices: ids E.., one sigmoid-gated weight
      ids[size_t(t) * ks + tid] = uint32_t(E + tid - k);
      scores[size_t(t) * ks + tid] = sigmoidf_(rs.vals[E]);
    }
    __syncthreads();
  }
}

// ---- cache-biased route (route_cuda.route / bias_probs) -------------------------------------------------------
//
// The reference's CacheBiasedMoE selection as one kernel (route_cuda.py:42-174 route, 306-416 bias_probs), on its
// own numeric contract: MLX's tie rule and output order (ties to the LARGER index, the k picks ascending, best
// last), the bias and budget arithmetic in the gates' dtype T, and the budget's two k-gate sums in MLX's
// row_reduce_simple order. One wavefront a row, one workgroup (T <= 16).

constexpr int kRouteMaxT = 16;
constexpr int kRouteMaxE = 1024;

struct RouteArgs {
  const void *gates;  // [T][E] in gdt: gates, or logits when softmax
  int gdt, T, E, k;
  const float *mask;      // [E], or nullptr: table mode, mask = 0 <= slot_of < lim
  const int32_t *slot_of;  // [E] (nullptr: no table, no rhs / ok)
  int lim;
  float lam, tau;
  int softmax, norm;
  uint32_t *inds;  // [T][k]
  uint32_t *ok;    // [1] or nullptr
  int32_t *rhs;    // [T][k] or nullptr
  void *scores;    // [T][k] in gdt, or nullptr
};

// x rounded to nearest even in dtype dt (the value as a float). x is the fp32 result of the step before; opaque()
// keeps the compiler from merging that step's multiply into the f16 conversion (one rounding in place of two)
__device__ __forceinline__ float round_dt(float x, int dt) {
  if (dt == LMOE_F16) return float(_Float16(opaque(x)));
  if (dt == LMOE_BF16) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return x;  // NaN stays
    u += 0x7FFFu + ((u >> 16) & 1u);
    return __uint_as_float(u & 0xFFFF0000u);
  }
  return x;
}

// The wave-uniform number of this wavefront's keys at or above c: one ballot (v_cmp into a scalar pair) and one
// scalar popcount a key slot. A lone wavefront issues a vector instruction every ~4 cycles, so the scalar unit's
// counts are the short form; lane-local counts summed on DPP took twice the instructions.
template <int NPL>
__device__ __forceinline__ int count_ge(const uint32_t (&key)[NPL], uint32_t c) {
  int cnt = 0;
#pragma unroll
  for (int j = 0; j < NPL; ++j) cnt += __popcll(__ballot(key[j] >= c));
  return cnt;
}

// OR and AND of every key of the wavefront (lanes past E hold key 0 and take part), as wave-uniform scalars
template <int NPL>
__device__ __forceinline__ void key_bits(const uint32_t (&key)[NPL], uint32_t *o, uint32_t *a) {
  uint32_t vo = 0u, va = ~0u;
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    vo |= key[j];
    va &= key[j];
  }
#define LMOE_OR_AND(ctrl)                                                          \
  vo |= uint32_t(__builtin_amdgcn_update_dpp(0, int(vo), ctrl, 0xF, 0xF, false)); \
  va &= uint32_t(__builtin_amdgcn_update_dpp(0, int(va), ctrl, 0xF, 0xF, false))
  LMOE_OR_AND(kDppXor1);
  LMOE_OR_AND(kDppXor2);
  LMOE_OR_AND(kDppHalfMirror);
  LMOE_OR_AND(kDppMirror);
#undef LMOE_OR_AND
  vo |= __builtin_bit_cast(uint32_t, lane_xor16(__builtin_bit_cast(float, vo)));
  va &= __builtin_bit_cast(uint32_t, lane_xor16(__builtin_bit_cast(float, va)));
  vo |= __builtin_bit_cast(uint32_t, lane_xor32(__builtin_bit_cast(float, vo)));
  va &= __builtin_bit_cast(uint32_t, lane_xor32(__builtin_bit_cast(float, va)));
  *o = __builtin_amdgcn_readfirstlane(vo);
  *a = __builtin_amdgcn_readfirstlane(va);
}

// Thresholds of the k largest keys of NS key sets: for each, the largest t with at least k keys >= t, by a bitwise
// search. Every key of a set agrees on the bits where OR == AND, and so does its k-th largest key; the search runs
// only over bits lo..hi, the lowest and highest bits where some set's keys differ (bf16 gates have 16 trailing zero
// bits), starting from AND's bits above hi and taking AND's bits below lo. A step outside a set's own range leaves
// its threshold as it is: the candidate equals it (a bit every key has) or exceeds every key (a bit none has), and
// a bit below the set's range is one every key has or none has. Kept rolled: the kernel runs its path once a
// launch, so code length matters more than loop overhead.
template <int NPL, int NS>
__device__ __forceinline__ void kth_keys(const uint32_t (*keys)[NPL], int k, uint32_t *thr) {
  uint32_t o[NS], an[NS], diff = 0u;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    key_bits<NPL>(keys[s], &o[s], &an[s]);
    diff |= o[s] ^ an[s];
  }
  if (diff == 0u) {  // every set's keys are all equal
#pragma unroll
    for (int s = 0; s < NS; ++s) thr[s] = an[s];
    return;
  }
  const int hi = 31 - __builtin_clz(diff), lo = __builtin_ctz(diff);
  const uint32_t upto_hi = (2u << hi) - 1u;  // bits 0..hi (hi = 31: all of them)
#pragma unroll
  for (int s = 0; s < NS; ++s) thr[s] = an[s] & ~upto_hi;
#pragma unroll 1
  for (int b = hi; b >= lo; --b) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const uint32_t cand = thr[s] | (1u << b);
      thr[s] = count_ge<NPL>(keys[s], cand) >= k ? cand : thr[s];
    }
  }
#pragma unroll
  for (int s = 0; s < NS; ++s) thr[s] |= an[s] & ((1u << lo) - 1u);
}

template <int NPL>
__device__ __forceinline__ void keys_of(const float (&v)[NPL], int E, uint32_t (&key)[NPL]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < NPL; ++j) key[j] = lane + 64 * j < E ? logit_key(v[j]) : 0u;
}

// Set bits of the wave mask m in lanes below this one (v_mbcnt_lo / v_mbcnt_hi)
__device__ __forceinline__ int lanes_below(uint64_t m) {
  return int(__builtin_amdgcn_mbcnt_hi(uint32_t(m >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(m), 0u)));
}

// Given the threshold thr of the k largest keys: the picks (ties at thr taken from the highest index down),
// compacted to LDS in index order, each one's rank among them by (key, index) descending, position k - 1 - rank.
template <int NPL>
__device__ __forceinline__ void pick_mlx(const uint32_t (&key)[NPL], uint32_t thr, int k, uint32_t *lds,
                                         uint32_t *idx, int *pos) {
  const int lane = threadIdx.x & 63;
  int n_gt = 0, n_eq = 0;
  uint64_t eqm[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    n_gt += __popcll(__ballot(key[j] > thr));
    eqm[j] = __ballot(key[j] == thr);
    n_eq += __popcll(eqm[j]);
  }
  const int need = k - n_gt;  // >= 1 ties at thr are taken, highest index first
  bool sel[NPL];
  if (n_eq == need) {  // the usual case: no surplus ties, every key >= thr is picked
#pragma unroll
    for (int j = 0; j < NPL; ++j) sel[j] = key[j] >= thr;
  } else {
    int eq_after = 0;  // ties at thr with a higher j
#pragma unroll
    for (int j = NPL - 1; j >= 0; --j) {
      const int tie = int((eqm[j] >> lane) & 1u);
      const int higher = __popcll(eqm[j]) - lanes_below(eqm[j]) - tie;  // ties in this slot at higher lanes
      sel[j] = key[j] > thr || (tie && eq_after + higher < need);
      eq_after += __popcll(eqm[j]);
    }
  }
  int sel_before = 0;
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const uint64_t selm = __ballot(sel[j]);
    const int p = sel_before + lanes_below(selm);
    if (sel[j] && p < 32) {  // k <= 32 picks; the bound keeps every write inside this wavefront's 64 dwords
      lds[p] = key[j];
      lds[32 + p] = uint32_t(lane + 64 * j);
    }
    sel_before += __popcll(selm);
  }
  const bool bad = sel_before != k;  // exactly k by construction; otherwise every id is 0xFFFFFFFF (no expert)
  __builtin_amdgcn_wave_barrier();
  if (lane < k) {
    const uint32_t my_key = lds[lane], my_idx = lds[32 + lane];
    int rank = 0;
    // four picks a step from 16-byte reads (lds is 16-byte aligned; entries past k are masked off)
#pragma unroll 1
    for (int q0 = 0; q0 < k; q0 += 4) {
      const u32x4 kq = *reinterpret_cast<const u32x4 *>(lds + q0);
      const u32x4 iq = *reinterpret_cast<const u32x4 *>(lds + 32 + q0);
#pragma unroll
      for (int c = 0; c < 4; ++c)
        rank += (q0 + c < k && (kq[c] > my_key || (kq[c] == my_key && iq[c] > my_idx))) ? 1 : 0;
    }
    *idx = bad ? 0xFFFFFFFFu : my_idx;
    *pos = bad ? lane : k - 1 - rank;
  }
  __builtin_amdgcn_wave_barrier();
}


// The k largest of v (expert lane + 64 j, j < NPL, E <= 64 NPL) by MLX's stable ascending sort read from the
// back: equal values go to the larger index. Lanes < k get an expert in *idx and its position in the ascending
// output (best at k - 1) in *pos. A 32-step bit search for the k-th largest key, then the keys above it and the
// highest-index keys equal to it, compacted into lds (64 dwords), ranked by (key, index) descending.
template <int NPL>
__device__ __forceinline__ void select_mlx(const float (&v)[NPL], int E, int k, uint32_t *lds, uint32_t *idx,
                                           int *pos) {
  uint32_t key[NPL];
  keys_of<NPL>(v, E, key);
  uint32_t thr;
  kth_keys<NPL, 1>(&key, k, &thr);
  pick_mlx<NPL>(key, thr, k, lds, idx, pos);
}

// The reference budget's sum of k values in T (route_cuda.py:36-37, 98-113): lane l < 32 adds positions l*N .. l*N+N-1
// from 0 in order (N = 16 / sizeof(T)), each add rounded to T, then the 32 lanes combine by xor 16, 8, 4, 2, 1.
// sv: the k values by position (LDS). Wave-uniform result.
__device__ __forceinline__ float budget_sum(const float *sv, int k, int dt) {
  const int lane = threadIdx.x & 63;
  const int n = dt == LMOE_F32 ? 4 : 8;
  float a = 0.0f;
  for (int i = 0; i < n; ++i) {
    const int j = (lane & 31) * n + i;
    a = round_dt(a + (j < k ? sv[j] : 0.0f), dt);
  }
  // the xor 16, 8, 4, 2, 1 partners without an LDS round trip, each the partner's exact value: permlane16 swap
  // (lane l ^ 16), row rotate by 8 (l ^ 8), then row rotate by 4 (lane l -/+ 4 mod 16 holds the value of l ^ 4,
  // since lanes l and l ^ 8 agree after the first two steps), quad permutes (l ^ 2, l ^ 1)
  a = round_dt(a + lane_xor16(a), dt);
  a = round_dt(a + LMOE_DPP(a, kDppRor8), dt);
  a = round_dt(a + LMOE_DPP(a, kDppRor4), dt);
  a = round_dt(a + LMOE_DPP(a, kDppXor2), dt);
  a = round_dt(a + LMOE_DPP(a, kDppXor1), dt);
  return lane_value(a, 0);
}

template <int NPL, int DT>
__device__ __forceinline__ void route_row(const RouteArgs &a, int r, float *gl, uint32_t *scr, float *sv, uint32_t *okf) {
  const int lane = threadIdx.x & 63;
  const int E = a.E, k = a.k, dt = DT;
  float g[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int e = min(lane + 64 * j, E - 1);
    g[j] = load_elt(a.gates, size_t(r) * E + e, dt);
  }
  if (a.softmax) {  // gates = T(exp(v - max) / sum), the sum over the row's experts
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < NPL; ++j)
      if (lane + 64 * j < E) mx = fmaxf(mx, g[j]);
    mx = wave_max(mx);
    float ex[NPL], sum = 0.0f;
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      ex[j] = lane + 64 * j < E ? expf(g[j] - mx) : 0.0f;
      sum += ex[j];
    }
    const float inv = 1.0f / wave_sum(sum);
#pragma unroll
    for (int j = 0; j < NPL; ++j) g[j] = round_dt(ex[j] * inv, dt);
  }
  float lmx = -INFINITY, lmn = INFINITY, m[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int e = lane + 64 * j;
    if (e < E) {
      gl[e] = g[j];
      lmx = fmaxf(lmx, g[j]);
      lmn = fminf(lmn, g[j]);
    }
    const int ec = min(e, E - 1);
    if (a.mask) {
      m[j] = a.mask[ec];
    } else {
      const int sl = a.slot_of[ec];
      m[j] = (sl >= 0 && sl < a.lim) ? 1.0f : 0.0f;
    }
  }
  lmx = wave_max(lmx);
  lmn = -wave_max(-lmn);
  const float spread = round_dt(lmx - lmn, dt);
  const float ls = round_dt(round_dt(a.lam, dt) * spread, dt);
  float rank[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) rank[j] = g[j] + ls * m[j];  // two roundings (no contraction in this library)
  uint32_t bi = 0, hi = 0;
  int bp = 0, hp = 0;
  bool back = false;
  if (a.tau > 0.0f) {  // both selections' searches in one loop, then the budget: honest mass against biased mass
    uint32_t ks[2][NPL], th[2];  // 0: the biased ranking's keys, 1: the honest gates'
    keys_of<NPL>(rank, E, ks[0]);
    keys_of<NPL>(g, E, ks[1]);
    kth_keys<NPL, 2>(ks, k, th);
    pick_mlx<NPL>(ks[0], th[0], k, scr, &bi, &bp);
    pick_mlx<NPL>(ks[1], th[1], k, scr, &hi, &hp);
    if (lane < k) {
      sv[hp] = gl[min(hi, uint32_t(E - 1))];
      sv[32 + bp] = gl[min(bi, uint32_t(E - 1))];
    }
    __builtin_amdgcn_wave_barrier();
    const float mh = budget_sum(sv, k, dt), mb = budget_sum(sv + 32, k, dt);
    back = round_dt(mh - mb, dt) > round_dt(round_dt(a.tau, dt) * mh, dt);
    __builtin_amdgcn_wave_barrier();
  } else {
    select_mlx<NPL>(rank, E, k, scr, &bi, &bp);
  }
  const uint32_t idx = min(back ? hi : bi, uint32_t(E - 1));  // always < E for finite gates; NaN rows stay in bounds
  const int p = back ? hp : bp;
  bool bad = false;
  if (lane < k) {
    a.inds[size_t(r) * k + p] = idx;
    if (a.slot_of) {
      const int sl = a.slot_of[idx];
      if (a.rhs) a.rhs[size_t(r) * k + p] = sl > 0 ? sl : 0;
      bad = sl < 0;
    }
  }
  if (__ballot(bad) != 0 && lane == 0) *okf = 0u;
  if (a.scores) {  // the picked gates, divided by their sum taken in position order from 0 in T when norm
    float sc = lane < k ? gl[idx] : 0.0f;
    if (a.norm) {
      if (lane < k) sv[p] = sc;
      __builtin_amdgcn_wave_barrier();
      float tot = 0.0f;
#pragma unroll 1
      for (int j = 0; j < k; ++j) tot = round_dt(tot + sv[j], dt);
      sc = round_dt(sc / tot, dt);
    }
    if (lane < k) store_elt(a.scores, size_t(r) * k + p, sc, dt);
  }
}

// One kernel per NPL (E <= 64 NPL) and gate dtype: the dtype's roundings fold to straight-line code, which keeps
// the path this one-wavefront-a-row kernel runs once a launch short (its instruction fetch is cold).
template <int NPL, int DT>
__global__ void __launch_bounds__(1024) k_route_bias(RouteArgs a) {
  __shared__ float gl[kRouteMaxT][64 * NPL];
  __shared__ __attribute__((aligned(16))) uint32_t scr[kRouteMaxT][64];
  __shared__ float sv[kRouteMaxT][64];
  __shared__ uint32_t okf;
  const int wave = threadIdx.x >> 6;
  if (threadIdx.x == 0) okf = 1u;
  __syncthreads();
  if (wave < a.T) route_row<NPL, DT>(a, wave, gl[wave], scr[wave], sv[wave], &okf);
  __syncthreads();
  if (threadIdx.x == 0 && a.ok) a.ok[0] = okf;
}

}  // namespace lmoe

using namespace lmoe;

static int topk_launch(const void *logits, int ldtype, int stride, int T, int E, int k, int norm, uint32_t *ids,
                       float *scores, hipStream_t st, const char *fn, const float *gate = nullptr, int m = 0) {
  LMOE_REQUIRE(dtype_ok(ldtype), LMOE_EINVAL, "%s: logits dtype %d is not F32, F16 or BF16", fn, ldtype);
  LMOE_REQUIRE(T >= 0 && E > 0 && E <= 64 * kMaxNpl, LMOE_ESHAPE, "%s: %d experts is outside 1..%d", fn, E,
               64 * kMaxNpl);
  LMOE_REQUIRE(k > 0 && k <= E && k <= 32, LMOE_ESHAPE, "%s: top-k %d is outside 1..min(E, 32)", fn, k);
  if (T == 0) return 0;
  LMOE_REQUIRE(logits && ids && scores, LMOE_EINVAL, "%s: null pointer", fn);
  const dim3 grid((T + 3) / 4), block(256);
  if (E <= 64)
    launch(k_router_topk<1>, grid, block, 0, st, logits, ldtype, stride, T, E, k, norm, ids, scores, gate, m);
  else if (E <= 128)
    launch(k_router_topk<2>, grid, block, 0, st, logits, ldtype, stride, T, E, k, norm, ids, scores, gate, m);
  else if (E <= 256)
    launch(k_router_topk<4>, grid, block, 0, st, logits, ldtype, stride, T, E, k, norm, ids, scores, gate, m);
  else if (E <= 512)
    launch(k_router_topk<8>, grid, block, 0, st, logits, ldtype, stride, T, E, k, norm, ids, scores, gate, m);
  else
    launch(k_router_topk<16>, grid, block, 0, st, logits, ldtype, stride, T, E, k, norm, ids, scores, gate, m);
  LMOE_LAUNCHED(fn);
  return 0;
}

extern "C" int lmoe_router_topk(const void *logits, int ldtype, int T, int E, int k, int norm, uint32_t *ids,
                                float *scores, void *stream) {
  return topk_launch(logits, ldtype, E, T, E, k, norm, ids, scores, (hipStream_t)stream, "lmoe_router_topk");
}

extern "C" int lmoe_topk_and_gemm_f16(const void *logits, int ldtype, int T, int E, int k, int norm, uint32_t *ids,
                                      float *scores, const void *x, int xdtype, long long n, void *xh, void *stream) {
  const char *fn = "lmoe_topk_and_gemm_f16";
  LMOE_REQUIRE(dtype_ok(ldtype) && dtype_ok(xdtype), LMOE_EINVAL, "%s: bad dtype", fn);
  LMOE_REQUIRE(T >= 0 && E > 0 && E <= 64 * kMaxNpl, LMOE_ESHAPE, "%s: %d experts is outside 1..%d", fn, E,
               64 * kMaxNpl);
  LMOE_REQUIRE(k > 0 && k <= E && k <= 32, LMOE_ESHAPE, "%s: top-k %d is outside 1..min(E, 32)", fn, k);
  LMOE_REQUIRE(n >= 0 && n % 32 == 0, LMOE_ESHAPE, "%s: length %lld is not a multiple of 32", fn, n);
  LMOE_REQUIRE(T == 0 || (logits && ids && scores), LMOE_EINVAL, "%s: null pointer", fn);
  LMOE_REQUIRE(n == 0 || (x && xh && aligned16(x) && aligned16(xh)), LMOE_EALIGN,
               "%s: x and xh must be given and 16-byte aligned", fn);
  const long long nb_conv = (n + 2047) / 2048, nb_topk = (T + 3) / 4;
  LMOE_REQUIRE(nb_conv + nb_topk < (1ll << 31), LMOE_ESHAPE, "%s: %lld workgroups", fn, nb_conv + nb_topk);
  if (nb_conv + nb_topk == 0) return 0;
  const dim3 grid(unsigned(nb_conv + nb_topk)), block(256);
  hipStream_t st = (hipStream_t)stream;
  _Float16 *out = static_cast<_Float16 *>(xh);
  const int nt = int(nb_topk);
  if (E <= 64)
    launch(k_topk_and_f16<1>, grid, block, 0, st, logits, ldtype, T, E, k, norm, ids, scores, nt, x, xdtype, n, out);
  else if (E <= 128)
    launch(k_topk_and_f16<2>, grid, block, 0, st, logits, ldtype, T, E, k, norm, ids, scores, nt, x, xdtype, n, out);
  else if (E <= 256)
    launch(k_topk_and_f16<4>, grid, block, 0, st, logits, ldtype, T, E, k, norm, ids, scores, nt, x, xdtype, n, out);
  else if (E <= 512)
    launch(k_topk_and_f16<8>, grid, block, 0, st, logits, ldtype, T, E, k, norm, ids, scores, nt, x, xdtype, n, out);
  else
    launch(k_topk_and_f16<16>, grid, block, 0, st, logits, ldtype, T, E, k, norm, ids, scores, nt, x, xdtype, n,
           out);
  LMOE_LAUNCHED(fn);
  return 0;
}

extern "C" int lmoe_router_topk_shared(const float *logits, int T, int E, int k, int norm, const float *gate, int m,
                                       uint32_t *ids, float *scores, void *stream) {
  const char *fn = "lmoe_router_topk_shared";
  LMOE_REQUIRE(m >= 1 && k + m <= 64, LMOE_ESHAPE, "%s: %d shared slices with top-%d", fn, m, k);
  LMOE_REQUIRE(T == 0 || gate, LMOE_EINVAL, "%s: null gate", fn);
  return topk_launch(logits, LMOE_F32, E, T, E, k, norm, ids, scores, (hipStream_t)stream, fn, gate, m);
}

extern "C" int lmoe_prep_x(const void *x, int xdtype, int rows, int H, int qtype, uint32_t *xprep, void *stream) {
  const char *fn = "lmoe_prep_x";
  LMOE_REQUIRE(dtype_ok(xdtype), LMOE_EINVAL, "%s: bad dtype", fn);
  LMOE_REQUIRE(qtype_ok(qtype), LMOE_ETYPE, "%s: ggml type %d is not supported (Q4_0 = 2, Q4_K = 12)", fn, qtype);
  LMOE_REQUIRE(rows >= 0 && H > 0 && H % 64 == 0, LMOE_ESHAPE, "%s: width %d is not a multiple of 64", fn, H);
  if (rows == 0) return 0;
  LMOE_REQUIRE(x && xprep, LMOE_EINVAL, "%s: null pointer", fn);
  const dim3 grid(((H / 64) * XS + 255) / 256, rows);
  if (qtype == LMOE_Q4_K)
    launch(k_prep_x<LMOE_Q4_K>, grid, dim3(256), 0, (hipStream_t)stream, x, xdtype, H, xprep);
  else
    launch(k_prep_x<LMOE_Q4_0>, grid, dim3(256), 0, (hipStream_t)stream, x, xdtype, H, xprep);
  LMOE_LAUNCHED(fn);
  return 0;
}

extern "C" int lmoe_router_gemv(const void *x, int xdtype, const void *wr, const void *wsg, int wdtype, int T, int H,
                                int E, float *logits, uint32_t *xprep, int qtype, void *stream) {
  const char *fn = "lmoe_router_gemv";
  LMOE_REQUIRE(dtype_ok(xdtype) && dtype_ok(wdtype), LMOE_EINVAL, "%s: bad dtype", fn);
  LMOE_REQUIRE(T > 0 && T <= kRouterMaxT, LMOE_ESHAPE, "%s: %d tokens is outside 1..%d", fn, T, kRouterMaxT);
  LMOE_REQUIRE(H > 0 && H % 64 == 0, LMOE_ESHAPE, "%s: hidden %d is not a multiple of 64", fn, H);
  LMOE_REQUIRE(E > 0, LMOE_ESHAPE, "%s: no experts", fn);
  LMOE_REQUIRE(!xprep || qtype_ok(qtype), LMOE_ETYPE, "%s: ggml type %d is not supported (Q4_0 = 2, Q4_K = 12)", fn,
               qtype);
  LMOE_REQUIRE(x && wr && logits, LMOE_EINVAL, "%s: null pointer", fn);
  LMOE_REQUIRE(aligned16(x) && aligned16(wr) && (!wsg || aligned16(wsg)), LMOE_EALIGN,
               "%s: x, wr and wsg must be 16-byte aligned", fn);
  LMOE_REQUIRE(H <= 8 * 256 * kRouterMaxNi, LMOE_ESHAPE, "%s: hidden %d is above the %d this kernel takes", fn, H,
               8 * 256 * kRouterMaxNi);
  const int rows = E + (wsg ? 1 : 0);
  const dim3 grid(rows + (xprep ? (T * (H / 64) + 3) / 4 : 0)), block(256);
  hipStream_t st = (hipStream_t)stream;
  if (wdtype == LMOE_F16)
    launch_router<LMOE_F16>(qtype, grid, block, st, x, xdtype, wr, wsg, T, H, E, logits, xprep);
  else if (wdtype == LMOE_BF16)
    launch_router<LMOE_BF16>(qtype, grid, block, st, x, xdtype, wr, wsg, T, H, E, logits, xprep);
  else
    launch_router<LMOE_F32>(qtype, grid, block, st, x, xdtype, wr, wsg, T, H, E, logits, xprep);
  LMOE_LAUNCHED(fn);
  return 0;
}

extern "C" int lmoe_router_gemv_topk(const void *x, int xdtype, const void *wr, const void *wsg, int wdtype, int T,
                                     int H, int E, int k, int norm, float *logits, uint32_t *ids, float *scores,
                                     uint32_t *xprep, int qtype, void *stream) {
  if (int rc = lmoe_router_gemv(x, xdtype, wr, wsg, wdtype, T, H, E, logits, xprep, qtype, stream)) return rc;
  return topk_launch(logits, LMOE_F32, E + (wsg ? 1 : 0), T, E, k, norm, ids, scores, (hipStream_t)stream,
                     "lmoe_router_gemv_topk");
}

extern "C" int lmoe_route_bias(const void *gates, int gdtype, int T, int E, int k, const float *mask,
                               const int32_t *slot_of, int lim, float lam, float tau, int softmax, int norm,
                               uint32_t *inds, uint32_t *ok, int32_t *rhs, void *scores, void *stream) {
  const char *fn = "lmoe_route_bias";
  LMOE_REQUIRE(dtype_ok(gdtype), LMOE_EINVAL, "%s: bad dtype", fn);
  LMOE_REQUIRE(T > 0 && T <= kRouteMaxT, LMOE_ESHAPE, "%s: %d rows is outside 1..%d", fn, T, kRouteMaxT);
  LMOE_REQUIRE(E > 0 && E <= kRouteMaxE && k > 0 && k <= 32 && k <= E, LMOE_ESHAPE,
               "%s: E = %d, k = %d (E <= %d, k <= 32)", fn, E, k, kRouteMaxE);
  LMOE_REQUIRE(lam >= 0.0f && tau >= 0.0f, LMOE_EINVAL, "%s: lam and tau must be >= 0", fn);
  LMOE_REQUIRE(gates && inds, LMOE_EINVAL, "%s: null pointer", fn);
  LMOE_REQUIRE(mask || slot_of, LMOE_EINVAL, "%s: give a mask or a slot table (table mode)", fn);
  LMOE_REQUIRE(slot_of || (!rhs && !ok), LMOE_EINVAL, "%s: rhs and ok need the slot table", fn);
  RouteArgs a{gates, gdtype, T, E, k, mask, slot_of, lim, lam, tau, softmax, norm, inds, ok, rhs, scores};
  const int npl = (E + 63) / 64;
  auto go = [&](auto kern) { launch(kern, dim3(1), dim3(64 * T), 0, (hipStream_t)stream, a); };
  auto by_npl = [&](auto dtc) {
    constexpr int D = decltype(dtc)::value;
    if (npl <= 1)
      go(k_route_bias<1, D>);
    else if (npl <= 2)
      go(k_route_bias<2, D>);
    else if (npl <= 4)
      go(k_route_bias<4, D>);
    else if (npl <= 8)
      go(k_route_bias<8, D>);
    else
      go(k_route_bias<16, D>);
  };
  if (a.gdt == LMOE_BF16)
    by_npl(std::integral_constant<int, LMOE_BF16>());
  else if (a.gdt == LMOE_F16)
    by_npl(std::integral_constant<int, LMOE_F16>());
  else
    by_npl(std::integral_constant<int, LMOE_F32>());
  LMOE_LAUNCHED(fn);
  return 0;
}

// Router rows a workgroup of k_router_rank: 1, 2, 4 or 8. More rows a workgroup mean fewer arrivals on the counter
// but less memory parallelism for the GEMV. LMOE_RANK_ROWS overrides the choice.
static int rank_rows(int rows) {
  static const int forced = [] {
    const char *v = getenv("LMOE_RANK_ROWS");
    const int n = v ? atoi(v) : 0;
    return (n == 1 || n == 2 || n == 4 || n == 8) ? n : 0;
  }();
  if (forced) return forced;
  return rows <= 160 ? 2 : 4;
}

extern "C" int lmoe_router_gemv_rank(const void *x, int xdtype, const void *wr, const void *wsg, int wdtype, int T,
                                     int H, int E, int k, int norm, int ks, float *logits, uint32_t *ids,
                                     float *scores, uint32_t *xprep, int qtype, uint32_t *sync, void *stream) {
  const char *fn = "lmoe_router_gemv_rank";
  LMOE_REQUIRE(dtype_ok(xdtype) && dtype_ok(wdtype), LMOE_EINVAL, "%s: bad dtype", fn);
  LMOE_REQUIRE(T > 0 && T <= kRouterMaxT, LMOE_ESHAPE, "%s: %d tokens is outside 1..%d", fn, T, kRouterMaxT);
  LMOE_REQUIRE(H > 0 && H % 64 == 0 && H <= 8 * 256 * kRouterMaxNi, LMOE_ESHAPE, "%s: hidden %d", fn, H);
  LMOE_REQUIRE(E > 0 && E <= kRankMaxE && k > 0 && k <= kRankMaxK && k <= E, LMOE_ESHAPE,
               "%s: top-%d of %d experts (E <= %d, k <= %d)", fn, k, E, kRankMaxE, kRankMaxK);
  LMOE_REQUIRE(ks == k || (ks > k && ks <= 64 && wsg), LMOE_EINVAL, "%s: %d slots a token for top-%d", fn, ks, k);
  LMOE_REQUIRE(!xprep || qtype_ok(qtype), LMOE_ETYPE, "%s: ggml type %d is not supported (Q4_0 = 2, Q4_K = 12)", fn,
               qtype);
  LMOE_REQUIRE(x && wr && logits && ids && scores && sync, LMOE_EINVAL, "%s: null pointer", fn);
  LMOE_REQUIRE(aligned16(x) && aligned16(wr) && (!wsg || aligned16(wsg)), LMOE_EALIGN,
               "%s: x, wr and wsg must be 16-byte aligned", fn);
  const int rows = E + (wsg ? 1 : 0);
  const int rr = rank_rows(rows);
  const int nr = (rows + rr - 1) / rr;
  const dim3 grid(nr + (xprep ? (T * (H / 64) + 3) / 4 : 0)), block(256);
  hipStream_t st = (hipStream_t)stream;
  const int ni = (H / 8 + 255) / 256;
  auto go = [&](auto wdc, auto tqc) {
    constexpr int WD = decltype(wdc)::value, TQ = decltype(tqc)::value;
    auto by_rr = [&](auto nic) {
      constexpr int NI = decltype(nic)::value;
      auto run = [&](auto kern) {
        launch(kern, grid, block, 0, st, x, xdtype, wr, wsg, T, H, E, k, norm, ks, logits, ids, scores, xprep, sync,
               nr);
      };
      if (rr == 1)
        run(k_router_rank<WD, TQ, NI, 1>);
      else if (rr == 2)
        run(k_router_rank<WD, TQ, NI, 2>);
      else if (rr == 4)
        run(k_router_rank<WD, TQ, NI, 4>);
      else
        run(k_router_rank<WD, TQ, NI, 8>);
    };
    if (ni <= 1)
      by_rr(std::integral_constant<int, 1>());
    else if (ni <= 2)
      by_rr(std::integral_constant<int, 2>());
    else
      by_rr(std::integral_constant<int, 4>());
  };
  auto by_q = [&](auto wdc) {
    if (qtype == LMOE_Q4_K)
      go(wdc, std::integral_constant<int, LMOE_Q4_K>());
    else
      go(wdc, std::integral_constant<int, LMOE_Q4_0>());
  };
  if (wdtype == LMOE_F16)
    by_q(std::integral_constant<int, LMOE_F16>());
  else if (wdtype == LMOE_BF16)
    by_q(std::integral_constant<int, LMOE_BF16>());
  else
    by_q(std::integral_constant<int, LMOE_F32>());
  LMOE_LAUNCHED(fn);
  return 0;
}
