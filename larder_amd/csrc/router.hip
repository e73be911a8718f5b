// Router: the gate GEMV (logits = x . Wr) and softmax + top-k.
//
// The reference runs the gate linear as an MLX matmul and the top-k in moe_probs, one 32-lane warp a row doing k
// rounds of shuffle argmax (route_cuda.py:193-254). Here:
//   * k_router_gemv spreads the E router rows over wavefronts (one row each, all T tokens), the row's weights
//     fetched with 16-byte loads while x is staged in LDS, and emits the prepared activation rows the expert
//     kernels read (lmoe_common.h), so no later kernel rearranges x again;
//   * k_router_topk takes k rounds of a wavefront argmax, one wavefront a token, its max and min-index reductions
//     on DPP and gfx950's permlane swaps rather than LDS shuffles.
// Selection is on the fp32 logits, larger first, ties to the lower expert index; scores are the softmax
// probabilities of the picked experts (max-subtracted, fp32), renormalised when asked.
#include "lmoe_common.h"

namespace lmoe {

constexpr int kMaxNpl = 16;  // logits a lane: E <= 64 * 16

// Four tokens a workgroup, one wavefront each.
template <int NPL>
__global__ void __launch_bounds__(256) k_router_topk(const void *logits, int ldt, int ld_stride, int T, int E,
                                                     int k, int norm, uint32_t *ids, float *scores) {
  __shared__ __attribute__((aligned(16))) uint32_t scr[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + wave;
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
  if (lane < k) {
    ids[size_t(t) * k + lane] = id;
    scores[size_t(t) * k + lane] = sc;
  }
}

constexpr int kRouterWaves = 4;
constexpr int kRouterMaxT = 16;
constexpr int kRouterMaxXs = 16384;  // T * H floats of x held in LDS
constexpr int kRouterNc = 16;        // 16-byte weight chunks a lane (H * element size <= 16 KiB)

// Each wavefront one router row (the last row the shared-expert gate when wsg is given) for all T tokens: its
// weight chunks load first, x is staged in LDS as f32 meanwhile. When xprep is given the workgroups also write
// the prepared activation rows for block type TQ, a slice of units each. WDT: the weights' element type.
template <int WDT, int TQ, int XB>
__global__ void __launch_bounds__(64 * kRouterWaves)
    k_router_gemv(const void *x, int xdt, const void *wr, const void *wsg, int T, int H, int E, float *logits,
                  uint32_t *xprep) {
  constexpr int EPC = WDT == LMOE_F32 ? 4 : 8;  // elements a 16-byte chunk
  __shared__ float xs[kRouterMaxXs];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rows = E + (wsg != nullptr ? 1 : 0);
  const int row = blockIdx.x * kRouterWaves + wave;
  const int nch = H / EPC;
  // x's 16-byte chunks (XB a thread, XB * 256 >= T H / elements a chunk) go out first, since they gate the LDS
  // staging; then the row's weights, needed only by the dot. No load is predicated (indices clamped; a wavefront
  // past the last row re-reads it), so each group issues back to back.
  const int epc = xdt == LMOE_F32 ? 4 : 8, nx = T * H / epc;
  const u32x4 *x4 = static_cast<const u32x4 *>(x);
  constexpr int NT = 64 * kRouterWaves;
  u32x4 xv[XB];
#pragma unroll
  for (int j = 0; j < XB; ++j) xv[j] = x4[min(int(threadIdx.x) + j * NT, nx - 1)];
  u32x4 w[kRouterNc];
  {
    const int rs = min(row, rows - 1);
    const u32x4 *src = reinterpret_cast<const u32x4 *>(rs < E ? static_cast<const char *>(wr) +
                                                                    size_t(rs) * H * (WDT == LMOE_F32 ? 4 : 2)
                                                              : static_cast<const char *>(wsg));
#pragma unroll
    for (int i = 0; i < kRouterNc; ++i) w[i] = __builtin_nontemporal_load(src + min(lane + 64 * i, nch - 1));
  }
  // x into LDS as f32
#pragma unroll
  for (int j = 0; j < XB; ++j) {
    const int q = threadIdx.x + j * NT;
    if (q >= nx) continue;
    const uint32_t u[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
    float *o = xs + q * epc;
    if (xdt == LMOE_F32) {
      *reinterpret_cast<float4 *>(o) =
          float4{__uint_as_float(u[0]), __uint_as_float(u[1]), __uint_as_float(u[2]), __uint_as_float(u[3])};
    } else {
      float f[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f[2 * i] = xdt == LMOE_F16 ? half_lo(u[i]) : __uint_as_float(u[i] << 16);
        f[2 * i + 1] = xdt == LMOE_F16 ? half_hi(u[i]) : __uint_as_float(u[i] & 0xFFFF0000u);
      }
      *reinterpret_cast<float4 *>(o) = float4{f[0], f[1], f[2], f[3]};
      *reinterpret_cast<float4 *>(o + 4) = float4{f[4], f[5], f[6], f[7]};
    }
  }
  __syncthreads();
  if (xprep) {  // prepared rows: units spread over the workgroups
    const int P = H / 64, units = T * P;
    const int per = (units + gridDim.x - 1) / gridDim.x;
    const int u0 = blockIdx.x * per, u1 = min(units, u0 + per);
    for (int idx = u0 * XS + threadIdx.x; idx < u1 * XS; idx += 64 * kRouterWaves) {
      const int u = idx / XS, dw = idx - u * XS, t = u / P, p = u - t * P;
      const float *xt = xs + t * H;
      xprep[size_t(u) * XS + dw] = prep_dword<TQ>([&](int i) { return xt[i]; }, p, dw);
    }
  }
  if (row >= rows) return;
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
  const int nx = T * H / (xdt == LMOE_F32 ? 4 : 8), xb = (nx + 64 * kRouterWaves - 1) / (64 * kRouterWaves);
  if (xb <= 1)
    launch(k_router_gemv<WDT, TQ, 1>, grid, block, 0, st, x, xdt, wr, wsg, T, H, E, logits, xprep);
  else if (xb <= 2)
    launch(k_router_gemv<WDT, TQ, 2>, grid, block, 0, st, x, xdt, wr, wsg, T, H, E, logits, xprep);
  else if (xb <= 4)
    launch(k_router_gemv<WDT, TQ, 4>, grid, block, 0, st, x, xdt, wr, wsg, T, H, E, logits, xprep);
  else if (xb <= 8)
    launch(k_router_gemv<WDT, TQ, 8>, grid, block, 0, st, x, xdt, wr, wsg, T, H, E, logits, xprep);
  else
    launch(k_router_gemv<WDT, TQ, 16>, grid, block, 0, st, x, xdt, wr, wsg, T, H, E, logits, xprep);
}

template <int WDT>
static void launch_router(int qt, dim3 grid, dim3 block, hipStream_t st, const void *x, int xdt, const void *wr,
                          const void *wsg, int T, int H, int E, float *logits, uint32_t *xprep) {
  if (qt == LMOE_Q4_K)
    launch_router_q<WDT, LMOE_Q4_K>(grid, block, st, x, xdt, wr, wsg, T, H, E, logits, xprep);
  else
    launch_router_q<WDT, LMOE_Q4_0>(grid, block, st, x, xdt, wr, wsg, T, H, E, logits, xprep);
}

}  // namespace lmoe

using namespace lmoe;

static int topk_launch(const void *logits, int ldtype, int stride, int T, int E, int k, int norm, uint32_t *ids,
                       float *scores, hipStream_t st, const char *fn) {
  LMOE_REQUIRE(dtype_ok(ldtype), LMOE_EINVAL, "%s: logits dtype %d is not F32, F16 or BF16", fn, ldtype);
  LMOE_REQUIRE(T >= 0 && E > 0 && E <= 64 * kMaxNpl, LMOE_ESHAPE, "%s: %d experts is outside 1..%d", fn, E,
               64 * kMaxNpl);
  LMOE_REQUIRE(k > 0 && k <= E && k <= 32, LMOE_ESHAPE, "%s: top-k %d is outside 1..min(E, 32)", fn, k);
  if (T == 0) return 0;
  LMOE_REQUIRE(logits && ids && scores, LMOE_EINVAL, "%s: null pointer", fn);
  const dim3 grid((T + 3) / 4), block(256);
  if (E <= 64)
    launch(k_router_topk<1>, grid, block, 0, st, logits, ldtype, stride, T, E, k, norm, ids, scores);
  else if (E <= 128)
    launch(k_router_topk<2>, grid, block, 0, st, logits, ldtype, stride, T, E, k, norm, ids, scores);
  else if (E <= 256)
    launch(k_router_topk<4>, grid, block, 0, st, logits, ldtype, stride, T, E, k, norm, ids, scores);
  else if (E <= 512)
    launch(k_router_topk<8>, grid, block, 0, st, logits, ldtype, stride, T, E, k, norm, ids, scores);
  else
    launch(k_router_topk<16>, grid, block, 0, st, logits, ldtype, stride, T, E, k, norm, ids, scores);
  LMOE_LAUNCHED(fn);
  return 0;
}

extern "C" int lmoe_router_topk(const void *logits, int ldtype, int T, int E, int k, int norm, uint32_t *ids,
                                float *scores, void *stream) {
  return topk_launch(logits, ldtype, E, T, E, k, norm, ids, scores, (hipStream_t)stream, "lmoe_router_topk");
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
    hipLaunchKernelGGL(k_prep_x<LMOE_Q4_K>, grid, dim3(256), 0, (hipStream_t)stream, x, xdtype, H, xprep);
  else
    hipLaunchKernelGGL(k_prep_x<LMOE_Q4_0>, grid, dim3(256), 0, (hipStream_t)stream, x, xdtype, H, xprep);
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
  LMOE_REQUIRE(size_t(T) * H <= size_t(kRouterMaxXs), LMOE_ESHAPE,
               "%s: %d tokens x hidden %d is above the %d activations this kernel stages", fn, T, H, kRouterMaxXs);
  LMOE_REQUIRE(size_t(H) * (wdtype == LMOE_F32 ? 4 : 2) <= size_t(kRouterNc) * 64 * 16, LMOE_ESHAPE,
               "%s: a router row of %d weights is above what a wavefront holds", fn, H);
  const int rows = E + (wsg ? 1 : 0);
  const dim3 grid((rows + kRouterWaves - 1) / kRouterWaves), block(64 * kRouterWaves);
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
