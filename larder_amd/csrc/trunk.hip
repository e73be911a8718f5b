// The trunk's 4-bit affine matmul of T bf16 rows: the reference's route_cuda.qmv_rows (route_cuda.py:460-541),
// which gives every row the bits of MLX 0.32.4's one-row qmv kernel while reading the weights once for all rows.
//
// Weights in MLX's affine 4-bit layout: w uint32 [N][K / 8] (element j of a word at bits 4j), scales and biases
// bf16 [N][K / G]; weight = q s + b. The arithmetic, kept step for step so the output bits match:
//   * a row is worked by 32 lanes; lane l takes elements idx = base + 16 l .. idx + 15, base = 0, 512, ...;
//   * its 16 weights in bf16: bf16(bf16(q s) + b);
//   * 16 bf16 accumulators a row of x, slot e = element idx + e, each step one bf16 fused multiply-add;
//   * the 16 slots summed in float32 in slot order, the xor butterfly 16, 8, 4, 2, 1 in float32, bf16 out.
// On gfx950 a 64-lane wavefront works two output rows, one a 32-lane half, so each half is exactly the reference's
// warp and the butterfly stays inside the half (shuffles of width 32).
//
// bf16 arithmetic runs in float32 with gfx950's v_cvt_pk_bf16_f32 (round to nearest even) for each rounding:
// products of two bf16 values are exact in float32; the sum of two bf16 values is exact unless their exponents
// are more than 16 apart, where the small one cannot reach a bf16 rounding boundary. A fused multiply-add is one
// float32 sum then one bf16 rounding; that double rounding equals the single rounding of the exact value except
// when the float32 sum sits exactly on a bf16 midpoint with a nonzero error, where the error (recovered by TwoSum)
// moves the sum off the midpoint first. (gfx950 has no bf16 fused multiply-add instruction.)
#include "lmoe_common.h"

namespace lmoe {

typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// both values rounded to bf16 by one v_cvt_pk_bf16_f32 (round to nearest even), back as float32
__device__ __forceinline__ void bf16r2(float &a, float &b) {
  const uint32_t u = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
  a = __uint_as_float(u << 16);
  b = __uint_as_float(u & 0xffff0000u);
}


// x w + a for bf16 values x, w, a as a float32 value whose round-to-nearest-even to bf16 is the single rounding
// of the exact value: the float32 sum s and its exact error e (TwoSum; the product is exact); when s sits exactly
// on a bf16 midpoint and e != 0, s moves one float32 ulp toward the exact value (it cannot cross another bf16
// rounding boundary), so the conversion rounds the way the exact value does.
__device__ __forceinline__ float fma_bf16_pre(float x, float w, float a) {
  const float p = x * w;  // exact
  const float s = p + a;
  const float bb = s - p;
  const float e = (p - (s - bb)) + (a - bb);  // s + e == p + a exactly
  const uint32_t u = __float_as_uint(s);
  const bool fix = (u & 0xffffu) == 0x8000u && e != 0.0f;
  const uint32_t step = ((__float_as_uint(e) ^ u) >> 31) ? 0xffffffffu : 1u;  // away from zero when signs agree
  return __uint_as_float(fix ? u + step : u);
}

// Grid ceil(N / 8), 256 threads: wavefront w's lanes 0-31 work output row 8 bx + 2 w, lanes 32-63 the next one.
// x [NR][K] bf16, out [NR][N] bf16. K % 16 == 0, G % 16 == 0, K % G == 0.
template <int NR>
__global__ void __launch_bounds__(256) k_qmv_rows(const uint16_t *x, const uint32_t *w, const uint16_t *scales,
                                                  const uint16_t *biases, int N, int K, int G, uint16_t *out) {
  const int lane = threadIdx.x & 63, l = lane & 31;
  const int row = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 2 + (lane >> 5);
  const int rr = row < N ? row : N - 1;  // a half past N works the last row again and stores nothing
  const uint32_t *wr = w + size_t(rr) * (K / 8);
  const uint16_t *sr = scales + size_t(rr) * (K / G), *br = biases + size_t(rr) * (K / G);
  float acc[NR][16];
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[r][e] = 0.0f;
  for (int base = 0; base < K; base += 512) {
    const int idx = base + 16 * l;
    if (idx >= K) break;
    const u32x2_t wv = *reinterpret_cast<const u32x2_t *>(wr + (idx >> 3));
    const float s = bf16_to_f32(sr[idx / G]), b = bf16_to_f32(br[idx / G]);
    float wd[16];
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const uint32_t byte = ((p < 4 ? wv[0] : wv[1]) >> (8 * (p & 3))) & 0xffu;
      float m0 = float(byte & 15u) * s, m1 = float(byte >> 4) * s;  // exact
      bf16r2(m0, m1);
      m0 += b;  // exact, or too far from a rounding boundary to matter
      m1 += b;
      bf16r2(m0, m1);
      wd[2 * p] = m0;
      wd[2 * p + 1] = m1;
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const u32x4 *xp = reinterpret_cast<const u32x4 *>(x + size_t(r) * K + idx);
      const u32x4 xa = xp[0], xc = xp[1];
      const uint32_t xs[8] = {xa[0], xa[1], xa[2], xa[3], xc[0], xc[1], xc[2], xc[3]};
#pragma unroll
      for (int p = 0; p < 8; ++p) {
        float s0 = fma_bf16_pre(__uint_as_float(xs[p] << 16), wd[2 * p], acc[r][2 * p]);
        float s1 = fma_bf16_pre(__uint_as_float(xs[p] & 0xffff0000u), wd[2 * p + 1], acc[r][2 * p + 1]);
        bf16r2(s0, s1);
        acc[r][2 * p] = s0;
        acc[r][2 * p + 1] = s1;
      }
    }
  }
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) s += acc[r][e];
#pragma unroll
    for (int m = 16; m > 0; m >>= 1) s += __shfl_xor(s, m, 32);
    if (l == 0 && row < N) out[size_t(r) * N + row] = f32_to_bf16(s);
  }
}

// out = bf16(silu(g) u) for bf16 g, u: one rounding of the float32 value (the shared expert's SwiGLU between its
// qmv_rows projections).
__global__ void __launch_bounds__(256) k_swiglu_bf16(const uint16_t *g, const uint16_t *u, long long n,
                                                     uint16_t *out) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  out[i] = f32_to_bf16(silu_mul(bf16_to_f32(g[i]), bf16_to_f32(u[i])));
}

}  // namespace lmoe

using namespace lmoe;

extern "C" int lmoe_swiglu_bf16(const void *g, const void *u, long long n, void *out, void *stream) {
  const char *fn = "lmoe_swiglu_bf16";
  LMOE_REQUIRE(n >= 0, LMOE_ESHAPE, "%s: bad size", fn);
  if (n == 0) return 0;
  LMOE_REQUIRE(g && u && out, LMOE_EINVAL, "%s: null pointer", fn);
  launch(k_swiglu_bf16, dim3(unsigned((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
         static_cast<const uint16_t *>(g), static_cast<const uint16_t *>(u), n, static_cast<uint16_t *>(out));
  LMOE_LAUNCHED(fn);
  return 0;
}

extern "C" int lmoe_qmv_rows(const void *x, int T, const uint32_t *w, const void *scales, const void *biases, int N,
                             int K, int group_size, void *out, void *stream) {
  const char *fn = "lmoe_qmv_rows";
  LMOE_REQUIRE(T >= 0, LMOE_ESHAPE, "%s: %d rows", fn, T);
  LMOE_REQUIRE(N > 0 && K > 0 && K % 16 == 0 && group_size > 0 && group_size % 16 == 0 && K % group_size == 0,
               LMOE_ESHAPE, "%s: K %d and group size %d must be multiples of 16, K of the group size", fn, K,
               group_size);
  if (T == 0) return 0;
  LMOE_REQUIRE(x && w && scales && biases && out, LMOE_EINVAL, "%s: null pointer", fn);
  LMOE_REQUIRE(aligned16(x) && (reinterpret_cast<uintptr_t>(w) & 7u) == 0, LMOE_EALIGN,
               "%s: x must be 16-byte aligned, w 8-byte aligned", fn);
  const dim3 grid(unsigned((N + 7) / 8));
  hipStream_t st = (hipStream_t)stream;
  // at most 8 rows a launch (their accumulators stay in registers); rows 8.. in a second pass over the weights,
  // which changes no bit (each row's arithmetic is its own)
  for (int r0 = 0; r0 < T; r0 += 8) {
    const int nr = T - r0 < 8 ? T - r0 : 8;
    const uint16_t *xr = static_cast<const uint16_t *>(x) + size_t(r0) * K;
    uint16_t *orow = static_cast<uint16_t *>(out) + size_t(r0) * N;
    auto go = [&](auto kern) {
      launch(kern, grid, dim3(256), 0, st, xr, w, static_cast<const uint16_t *>(scales),
             static_cast<const uint16_t *>(biases), N, K, group_size, orow);
    };
    switch (nr) {
      case 1: go(k_qmv_rows<1>); break;
      case 2: go(k_qmv_rows<2>); break;
      case 3: go(k_qmv_rows<3>); break;
      case 4: go(k_qmv_rows<4>); break;
      case 5: go(k_qmv_rows<5>); break;
      case 6: go(k_qmv_rows<6>); break;
      case 7: go(k_qmv_rows<7>); break;
      default: go(k_qmv_rows<8>); break;
    }
    LMOE_LAUNCHED(fn);
  }
  return 0;
}
