// Router: softmax + top-k, one wavefront per token (the reference's moe_probs runs one 32-lane warp a row,
// route_cuda.py:193-254; here a 64-lane wavefront holds E <= 1024 logits as 16 registers a lane).
//
// Selection is made on the fp32 logits, larger first, equal values ordered by the lower expert index; the
// scores are the softmax probabilities of the picked experts (max-subtracted, fp32), renormalised when asked.
#include <cfloat>

#include "lmoe_common.h"

namespace lmoe {

constexpr int kMaxNpl = 16;  // logits a lane: E <= 64 * 16

// One wavefront: row[0..E) -> ids[0..k) best first, scores[0..k).
template <typename Load>
__device__ __forceinline__ void topk_wave(Load ld, int E, int k, int norm, uint32_t *ids, float *scores) {
  const int lane = threadIdx.x & 63;
  float v[kMaxNpl];
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < kMaxNpl; ++j) {
    const int i = lane + 64 * j;
    v[j] = i < E ? ld(i) : -INFINITY;
    m = fmaxf(m, v[j]);
  }
  m = wave_max(m);
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < kMaxNpl; ++j)
    if (lane + 64 * j < E) s += __expf(v[j] - m);
  s = wave_sum(s);
  uint32_t taken = 0;
  float mine = 0.0f;
  uint32_t my_id = 0;
  for (int r = 0; r < k; ++r) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < kMaxNpl; ++j) {
      const int i = lane + 64 * j;
      if (i < E && !((taken >> j) & 1u) && (v[j] > bv || (v[j] == bv && i < bi))) {
        bv = v[j];
        bi = i;
      }
    }
#pragma unroll
    for (int msk = 32; msk > 0; msk >>= 1) {
      const float ov = __shfl_xor(bv, msk, 64);
      const int oi = __shfl_xor(bi, msk, 64);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if ((bi & 63) == lane) taken |= 1u << ((bi >> 6) & 31);
    if (lane == r) {
      my_id = uint32_t(bi);
      mine = __expf(bv - m) / s;
    }
  }
  if (norm) {
    float tot = 0.0f;
    // the k picked probabilities summed in pick order (lane 0 reads them one by one)
    for (int r = 0; r < k; ++r) tot += __shfl(mine, r, 64);
    mine = mine / tot;
  }
  if (lane < k) {
    ids[lane] = my_id;
    scores[lane] = mine;
  }
}

__global__ void __launch_bounds__(256) k_router_topk(const void *logits, int ldt, int T, int E, int k, int norm,
                                                     uint32_t *ids, float *scores) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const size_t base = size_t(t) * E;
  topk_wave([&](int i) { return load_elt(logits, base + i, ldt); }, E, k, norm, ids + size_t(t) * k,
            scores + size_t(t) * k);
}

constexpr int kRouterWaves = 4;
constexpr int kRouterMaxT = 16;
constexpr int kRouterMaxXs = 16384;  // T * H floats of x held in LDS
constexpr int kRouterNc = 16;        // 16-byte weight chunks a lane (H * element size <= 16 KiB)

// Each wavefront one router row (the last row the shared-expert gate when wsg is given) for all T tokens: its
// weight chunks load first, x is staged in LDS as f32 meanwhile; then the last workgroup to finish runs the top-k
// of every token and returns the counter to zero for the next launch. WDT: the weights' element type.
template <int WDT>
__global__ void __launch_bounds__(64 * kRouterWaves)
    k_router_gemv(const void *x, int xdt, const void *wr, const void *wsg, int T, int H, int E, int k, int norm,
                  float *logits, uint32_t *ids, float *scores, uint32_t *counter) {
  constexpr int EPC = WDT == LMOE_F32 ? 4 : 8;  // elements a 16-byte chunk
  __shared__ float xs[kRouterMaxXs];
  __shared__ int last;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rows = E + (wsg != nullptr ? 1 : 0);
  const int row = blockIdx.x * kRouterWaves + wave;
  const int nch = H / EPC;
  u32x4 w[kRouterNc];
  if (row < rows) {
    const u32x4 *src = reinterpret_cast<const u32x4 *>(row < E ? static_cast<const char *>(wr) +
                                                                     size_t(row) * H * (WDT == LMOE_F32 ? 4 : 2)
                                                               : static_cast<const char *>(wsg));
#pragma unroll
    for (int i = 0; i < kRouterNc; ++i) {
      const int c = lane + 64 * i;
      if (c < nch) w[i] = __builtin_nontemporal_load(src + c);
    }
  }
  for (int i = threadIdx.x; i < T * H; i += 64 * kRouterWaves) xs[i] = load_elt(x, i, xdt);
  __syncthreads();
  if (row < rows) {
    float acc[kRouterMaxT];
#pragma unroll
    for (int t = 0; t < kRouterMaxT; ++t) acc[t] = 0.0f;
#pragma unroll
    for (int i = 0; i < kRouterNc; ++i) {
      const int c = lane + 64 * i;
      if (c < nch) {
        float wv[EPC];
        const uint32_t u[4] = {w[i].x, w[i].y, w[i].z, w[i].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (WDT == LMOE_F32) {
            wv[j] = __uint_as_float(u[j]);
          } else if (WDT == LMOE_F16) {
            wv[2 * j] = half_lo(u[j]);
            wv[2 * j + 1] = half_hi(u[j]);
          } else {
            wv[2 * j] = __uint_as_float(u[j] << 16);
            wv[2 * j + 1] = __uint_as_float(u[j] & 0xFFFF0000u);
          }
        }
        for (int t = 0; t < T; ++t) {
          const float *xt = xs + t * H + c * EPC;
#pragma unroll
          for (int j = 0; j < EPC; ++j) acc[t] = fmaf(xt[j], wv[j], acc[t]);
        }
      }
    }
#pragma unroll
    for (int t = 0; t < kRouterMaxT; ++t) {
      if (t < T) {
        const float v = wave_sum(acc[t]);
        if (lane == 0) logits[size_t(t) * rows + row] = v;
      }
    }
  }
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) last = atomicAdd(counter, 1u) == gridDim.x - 1;
  __syncthreads();
  if (!last) return;
  __threadfence();
  for (int t = wave; t < T; t += kRouterWaves) {
    const float *row_l = logits + size_t(t) * rows;
    topk_wave([&](int i) { return __builtin_nontemporal_load(row_l + i); }, E, k, norm, ids + size_t(t) * k,
              scores + size_t(t) * k);
  }
  if (threadIdx.x == 0) atomicExch(counter, 0u);
}

}  // namespace lmoe

using namespace lmoe;

extern "C" int lmoe_router_topk(const void *logits, int ldtype, int T, int E, int k, int norm, uint32_t *ids,
                                float *scores, void *stream) {
  LMOE_REQUIRE(dtype_ok(ldtype), LMOE_EINVAL, "lmoe_router_topk: logits dtype %d is not F32, F16 or BF16", ldtype);
  LMOE_REQUIRE(T >= 0 && E > 0 && E <= 64 * kMaxNpl, LMOE_ESHAPE,
               "lmoe_router_topk: %d experts is outside 1..%d", E, 64 * kMaxNpl);
  LMOE_REQUIRE(k > 0 && k <= E && k <= 32, LMOE_ESHAPE, "lmoe_router_topk: top-k %d is outside 1..min(E, 32)", k);
  if (T == 0) return 0;
  LMOE_REQUIRE(logits && ids && scores, LMOE_EINVAL, "lmoe_router_topk: null pointer");
  hipLaunchKernelGGL(k_router_topk, dim3((T + 3) / 4), dim3(256), 0, (hipStream_t)stream, logits, ldtype, T, E, k,
                     norm, ids, scores);
  LMOE_LAUNCHED("lmoe_router_topk");
  return 0;
}

extern "C" size_t lmoe_router_workspace_bytes(void) { return 256; }

extern "C" int lmoe_router_gemv_topk(const void *x, int xdtype, const void *wr, const void *wsg, int wdtype, int T,
                                     int H, int E, int k, int norm, float *logits, uint32_t *ids, float *scores,
                                     void *ws, void *stream) {
  LMOE_REQUIRE(dtype_ok(xdtype) && dtype_ok(wdtype), LMOE_EINVAL, "lmoe_router_gemv_topk: bad dtype");
  LMOE_REQUIRE(T > 0 && T <= kRouterMaxT, LMOE_ESHAPE, "lmoe_router_gemv_topk: %d tokens is outside 1..%d", T,
               kRouterMaxT);
  LMOE_REQUIRE(H > 0 && H % 64 == 0, LMOE_ESHAPE, "lmoe_router_gemv_topk: hidden %d is not a multiple of 64", H);
  LMOE_REQUIRE(E > 0 && E <= 64 * kMaxNpl, LMOE_ESHAPE, "lmoe_router_gemv_topk: %d experts is outside 1..%d", E,
               64 * kMaxNpl);
  LMOE_REQUIRE(k > 0 && k <= E && k <= 32, LMOE_ESHAPE, "lmoe_router_gemv_topk: top-k %d is outside 1..min(E, 32)",
               k);
  LMOE_REQUIRE(x && wr && logits && ids && scores && ws, LMOE_EINVAL, "lmoe_router_gemv_topk: null pointer");
  LMOE_REQUIRE(aligned16(wr) && (!wsg || aligned16(wsg)), LMOE_EALIGN,
               "lmoe_router_gemv_topk: wr and wsg must be 16-byte aligned");
  LMOE_REQUIRE(size_t(T) * H <= size_t(kRouterMaxXs), LMOE_ESHAPE,
               "lmoe_router_gemv_topk: %d tokens x hidden %d is above the %d activations this kernel stages", T, H,
               kRouterMaxXs);
  LMOE_REQUIRE(size_t(H) * (wdtype == LMOE_F32 ? 4 : 2) <= size_t(kRouterNc) * 64 * 16, LMOE_ESHAPE,
               "lmoe_router_gemv_topk: a router row of %d weights is above what a wavefront holds", H);
  const int rows = E + (wsg ? 1 : 0);
  const dim3 grid((rows + kRouterWaves - 1) / kRouterWaves), block(64 * kRouterWaves);
  hipStream_t st = (hipStream_t)stream;
  uint32_t *ctr = static_cast<uint32_t *>(ws);
  if (wdtype == LMOE_F16)
    hipLaunchKernelGGL(k_router_gemv<LMOE_F16>, grid, block, 0, st, x, xdtype, wr, wsg, T, H, E, k, norm, logits, ids,
                       scores, ctr);
  else if (wdtype == LMOE_BF16)
    hipLaunchKernelGGL(k_router_gemv<LMOE_BF16>, grid, block, 0, st, x, xdtype, wr, wsg, T, H, E, k, norm, logits,
                       ids, scores, ctr);
  else
    hipLaunchKernelGGL(k_router_gemv<LMOE_F32>, grid, block, 0, st, x, xdtype, wr, wsg, T, H, E, k, norm, logits, ids,
                       scores, ctr);
  LMOE_LAUNCHED("lmoe_router_gemv_topk");
  return 0;
}
