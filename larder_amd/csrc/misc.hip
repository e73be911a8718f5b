// Smaller kernels around the path: the weighted combine of grouped rows, the dequant of whole experts, and a
// Q4_0 quantizer used to build synthetic packs on the device.
#include "lmoe_common.h"

namespace lmoe {

// out[t][n] = sum_j scores[t][j] y[inv[t k + j]][n] (+ sigmoid(gate) shared) (+ residual), in that order of
// additions; VEC: 8 consecutive n a thread (H % 8 == 0, aligned rows), grid (ceil(H / 2048), T); else one n a
// thread, grid (ceil(H / 256), T).
template <bool VEC>
__global__ void __launch_bounds__(256)
    k_combine_sorted(const void *y, int ydt, const uint32_t *inv, const float *scores, int k, int H,
                     const float *shared, const float *gate, int gate_stride, const void *residual, int rdt,
                     void *out, int odt) {
  const int t = blockIdx.y;
  constexpr int NV = VEC ? 8 : 1;
  const int n = (blockIdx.x * 256 + threadIdx.x) * NV;
  if (n >= H) return;
  float acc[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) acc[i] = 0.0f;
  for (int j = 0; j < k; ++j) {
    const size_t row = inv[size_t(t) * k + j];
    const float s = scores ? scores[size_t(t) * k + j] : 1.0f;
    float v[NV];
    if (VEC)
      load8(y, row * H + n, ydt, v);
    else
      v[0] = load_elt(y, row * H + n, ydt);
#pragma unroll
    for (int i = 0; i < NV; ++i) acc[i] = fmaf(s, v[i], acc[i]);
  }
  const size_t o = size_t(t) * H + n;
  if (shared) {
    const float gs = sigmoidf_(gate[size_t(t) * gate_stride]);
#pragma unroll
    for (int i = 0; i < NV; ++i) acc[i] += gs * shared[o + i];
  }
  if (residual) {
    float v[NV];
    if (VEC)
      load8(residual, o, rdt, v);
    else
      v[0] = load_elt(residual, o, rdt);
#pragma unroll
    for (int i = 0; i < NV; ++i) acc[i] += v[i];
  }
  if (VEC)
    store8(out, o, odt, acc);
  else
    store_elt(out, o, acc[0], odt);
}

// One thread a 64-weight unit of one row of one expert: q[c][r][64 u .. 64 u + 63].
template <int TQ>
__global__ void __launch_bounds__(256) k_dequant(const uint8_t *buf, int n_experts, int rows, int cols,
                                                 const uint32_t *slots, int n, void *q, int odt) {
  const int P = cols / 64;
  const size_t g = size_t(blockIdx.x) * 256 + threadIdx.x;
  if (g >= size_t(n) * rows * P) return;
  const int u = int(g % P);
  const size_t rc = g / P;
  const int r = int(rc % rows), c = int(rc / rows);
  const uint32_t e = slots[c];
  const size_t o = (size_t(c) * rows + r) * cols + 64 * size_t(u);
  if (e >= uint32_t(n_experts)) {
    for (int i = 0; i < 64; ++i) store_elt(q, o + i, 0.0f, odt);
    return;
  }
  const uint8_t *row = buf + (size_t(e) * rows + r) * (size_t(36) * P);
  if (TQ == LMOE_Q4_0) {
    for (int b = 0; b < 2; ++b) {
      const uint8_t *blk = row + 36 * u + 18 * b;
      const float d = float(__builtin_bit_cast(_Float16, uint16_t(blk[0] | (blk[1] << 8))));
      for (int j = 0; j < 16; ++j) {
        const uint32_t v = blk[2 + j];
        store_elt(q, o + 32 * b + j, float(int(v & 15u) - 8) * d, odt);
        store_elt(q, o + 32 * b + 16 + j, float(int(v >> 4) - 8) * d, odt);
      }
    }
  } else {
    const uint32_t *sb = reinterpret_cast<const uint32_t *>(row + 144 * (u >> 2));
    const int c4 = u & 3;
    const float d = half_lo(sb[0]), dmin = half_hi(sb[0]);
    float sc0, m0, sc1, m1;
    k4_scale_min(sb[1], sb[2], sb[3], 2 * c4, &sc0, &m0);
    k4_scale_min(sb[1], sb[2], sb[3], 2 * c4 + 1, &sc1, &m1);
    const float d1 = d * sc0, n1 = dmin * m0, d2 = d * sc1, n2 = dmin * m1;
    const uint8_t *qs = row + 144 * (u >> 2) + 16 + 32 * c4;
    for (int l = 0; l < 32; ++l) {
      const uint32_t v = qs[l];
      store_elt(q, o + l, d1 * float(v & 15u) - n1, odt);
      store_elt(q, o + 32 + l, d2 * float(v >> 4) - n2, odt);
    }
  }
}

// ggml's quantize_row_q4_0_ref for one 32-weight block a thread, every step rounded on its own (the library is
// built with -ffp-contract=off: a fused x * id + 8.5 can truncate differently, and a multiply folded into the f16
// conversion as a mixed FMA with a +0 addend would turn d = -0 into +0).
__global__ void __launch_bounds__(256) k_quantize_q4_0(const void *w, int wdt, long long nblocks, uint8_t *out) {
  const long long b = (long long)blockIdx.x * 256 + threadIdx.x;
  if (b >= nblocks) return;
  float v[32];
  float amax = 0.0f, mx = 0.0f;
  for (int j = 0; j < 32; ++j) {
    v[j] = load_elt(w, size_t(b) * 32 + j, wdt);
    if (amax < fabsf(v[j])) {
      amax = fabsf(v[j]);
      mx = v[j];
    }
  }
  const float d = mx / -8.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  uint8_t *o = out + size_t(b) * 18;
  // the backend folds this conversion with the multiply above into a mixed FMA with a +0 addend, which drops the
  // sign of d = -0 (max = 0); the sign bit is restored from d itself
  const uint16_t dh = __builtin_bit_cast(uint16_t, _Float16(d)) | uint16_t((__float_as_uint(d) >> 16) & 0x8000u);
  o[0] = uint8_t(dh & 0xFF);
  o[1] = uint8_t(dh >> 8);
  for (int j = 0; j < 16; ++j) {
    const int q0 = min(15, int(int8_t(v[j] * id + 8.5f)));
    const int q1 = min(15, int(int8_t(v[j + 16] * id + 8.5f)));
    o[2 + j] = uint8_t(q0 | (q1 << 4));
  }
}

// One thread a Q4_K super-block of 256 weights (8 sub-blocks of 32), by a plain min/scale fit with no counterpart in
// ggml or the reference (which only read packs): sub-block j gets scale (max - min) / 15 and min -min(x, 0); the
// super-block's d and dmin are the largest of those over 63 (stored f16, round to nearest even); the 6-bit sc_j,
// m_j round (half to even) against the stored d, dmin; each weight takes q = clip(rint((x + dmin m_j) / (d sc_j)),
// 0, 15). Scales pack as ggml's get_scale_min_k4 reads them. Every step rounds on its own (no contraction).
__global__ void __launch_bounds__(256) k_quantize_q4_k(const void *w, int wdt, long long nblocks, uint8_t *out) {
  const long long b = (long long)blockIdx.x * 256 + threadIdx.x;
  if (b >= nblocks) return;
  const size_t base = size_t(b) * 256;
  float scale[8], mins[8];
  for (int j = 0; j < 8; ++j) {
    float lo = 0.0f, hi = -INFINITY;
    for (int i = 0; i < 32; ++i) {
      const float v = load_elt(w, base + 32 * j + i, wdt);
      lo = fminf(lo, v);
      hi = fmaxf(hi, v);
    }
    scale[j] = (hi - lo) / 15.0f;
    mins[j] = -lo;  // -0 when the sub-block has no negative weight
  }
  // maxima seeded with the first sub-block, so an all -0 set of mins keeps its sign (stored dmin = -0)
  float smax = scale[0], mmax = mins[0];
  for (int j = 1; j < 8; ++j) {
    smax = fmaxf(smax, scale[j]);
    mmax = fmaxf(mmax, mins[j]);
  }
  const float dq = smax / 63.0f, mq = mmax / 63.0f;
  const _Float16 d16 = _Float16(dq), m16 = _Float16(mq);
  const float d = float(d16), dm = float(m16);
  uint32_t sc[8], m[8];
  for (int j = 0; j < 8; ++j) {
    sc[j] = d > 0.0f ? uint32_t(fminf(fmaxf(rintf(scale[j] / d), 0.0f), 63.0f)) : 0u;
    m[j] = dm > 0.0f ? uint32_t(fminf(fmaxf(rintf(mins[j] / dm), 0.0f), 63.0f)) : 0u;
  }
  uint8_t *o = out + size_t(b) * 144;
  const uint16_t db = __builtin_bit_cast(uint16_t, d16), mb = __builtin_bit_cast(uint16_t, m16);
  o[0] = uint8_t(db & 0xFF);
  o[1] = uint8_t(db >> 8);
  o[2] = uint8_t(mb & 0xFF);
  o[3] = uint8_t(mb >> 8);
  for (int j = 0; j < 4; ++j) {
    o[4 + j] = uint8_t((sc[j] & 63u) | ((sc[j + 4] >> 4) << 6));
    o[8 + j] = uint8_t((m[j] & 63u) | ((m[j + 4] >> 4) << 6));
    o[12 + j] = uint8_t((sc[j + 4] & 15u) | ((m[j + 4] & 15u) << 4));
  }
  // sub-blocks 2c (low nibbles) and 2c + 1 (high nibbles) share qs bytes 32c .. 32c + 31
  for (int c = 0; c < 4; ++c) {
    const float dj0 = d * float(sc[2 * c]), mj0 = dm * float(m[2 * c]);
    const float dj1 = d * float(sc[2 * c + 1]), mj1 = dm * float(m[2 * c + 1]);
    for (int i = 0; i < 32; ++i) {
      const float x0 = load_elt(w, base + 64 * c + i, wdt), x1 = load_elt(w, base + 64 * c + 32 + i, wdt);
      const uint32_t q0 = dj0 > 0.0f ? uint32_t(fminf(fmaxf(rintf((x0 + mj0) / dj0), 0.0f), 15.0f)) : 0u;
      const uint32_t q1 = dj1 > 0.0f ? uint32_t(fminf(fmaxf(rintf((x1 + mj1) / dj1), 0.0f), 15.0f)) : 0u;
      o[16 + 32 * c + i] = uint8_t(q0 | (q1 << 4));
    }
  }
}

}  // namespace lmoe

using namespace lmoe;

extern "C" int lmoe_combine_sorted(const void *y, int ydtype, const uint32_t *inv, const float *scores, int T, int k,
                                   int H, const float *shared, const float *gate, int gate_stride,
                                   const void *residual, int rdtype, void *out, int odtype, void *stream) {
  const char *fn = "lmoe_combine_sorted";
  LMOE_REQUIRE(dtype_ok(ydtype) && dtype_ok(odtype) && (!residual || dtype_ok(rdtype)), LMOE_EINVAL,
               "%s: bad dtype", fn);
  LMOE_REQUIRE(T >= 0 && k > 0 && H > 0, LMOE_ESHAPE, "%s: bad shape", fn);
  LMOE_REQUIRE(!shared == !gate, LMOE_EINVAL, "%s: shared and gate go together", fn);
  if (T == 0) return 0;
  LMOE_REQUIRE(y && inv && out, LMOE_EINVAL, "%s: null pointer", fn);
  const bool vec = H % 8 == 0 && aligned16(y) && aligned16(out) && (!residual || aligned16(residual)) &&
                   (ydtype != LMOE_F32 || (reinterpret_cast<uintptr_t>(y) & 31u) == 0);
  if (vec)
    launch(k_combine_sorted<true>, dim3((H + 2047) / 2048, T), dim3(256), 0, (hipStream_t)stream, y, ydtype, inv,
           scores, k, H, shared, gate, gate_stride, residual, rdtype, out, odtype);
  else
    launch(k_combine_sorted<false>, dim3((H + 255) / 256, T), dim3(256), 0, (hipStream_t)stream, y, ydtype, inv,
           scores, k, H, shared, gate, gate_stride, residual, rdtype, out, odtype);
  LMOE_LAUNCHED(fn);
  return 0;
}

extern "C" int lmoe_dequant(const uint8_t *buf, int type, int n_experts, int rows, int cols, const uint32_t *slots,
                            int n, void *q, int odtype, void *stream) {
  const char *fn = "lmoe_dequant";
  if (!qtype_ok(type)) {
    LMOE_REQUIRE(n == 0 || slots, LMOE_EINVAL, "%s: null pointer", fn);
    return dequant_any(fn, buf, type, n_experts, rows, cols, slots, n, q, odtype, 0, (hipStream_t)stream);
  }
  LMOE_REQUIRE(dtype_ok(odtype), LMOE_EINVAL, "%s: bad dtype", fn);
  LMOE_REQUIRE(rows > 0 && cols > 0 && cols % block_weights(type) == 0 && cols % 64 == 0 && n >= 0, LMOE_ESHAPE,
               "%s: row length %d is not a multiple of %d", fn, cols, type == LMOE_Q4_K ? 256 : 64);
  if (n == 0) return 0;
  LMOE_REQUIRE(buf && slots && q, LMOE_EINVAL, "%s: null pointer", fn);
  LMOE_REQUIRE(type != LMOE_Q4_K || aligned4(buf), LMOE_EALIGN, "%s: Q4_K buffer must be 4-byte aligned", fn);
  const size_t units = size_t(n) * rows * (cols / 64);
  const dim3 grid(unsigned((units + 255) / 256));
  if (type == LMOE_Q4_0)
    hipLaunchKernelGGL(k_dequant<LMOE_Q4_0>, grid, dim3(256), 0, (hipStream_t)stream, buf, n_experts, rows, cols,
                       slots, n, q, odtype);
  else
    hipLaunchKernelGGL(k_dequant<LMOE_Q4_K>, grid, dim3(256), 0, (hipStream_t)stream, buf, n_experts, rows, cols,
                       slots, n, q, odtype);
  LMOE_LAUNCHED(fn);
  return 0;
}

extern "C" int lmoe_quantize_q4_0(const void *w, int wdtype, long long rows, int cols, uint8_t *out, void *stream) {
  const char *fn = "lmoe_quantize_q4_0";
  LMOE_REQUIRE(dtype_ok(wdtype), LMOE_EINVAL, "%s: bad dtype", fn);
  LMOE_REQUIRE(rows >= 0 && cols > 0 && cols % 32 == 0, LMOE_ESHAPE, "%s: row length %d is not a multiple of 32", fn,
               cols);
  const long long nb = rows * (cols / 32);
  if (nb == 0) return 0;
  LMOE_REQUIRE(w && out, LMOE_EINVAL, "%s: null pointer", fn);
  hipLaunchKernelGGL(k_quantize_q4_0, dim3(unsigned((nb + 255) / 256)), dim3(256), 0, (hipStream_t)stream, w, wdtype,
                     nb, out);
  LMOE_LAUNCHED(fn);
  return 0;
}

extern "C" int lmoe_quantize_q4_k(const void *w, int wdtype, long long rows, int cols, uint8_t *out, void *stream) {
  const char *fn = "lmoe_quantize_q4_k";
  LMOE_REQUIRE(dtype_ok(wdtype), LMOE_EINVAL, "%s: bad dtype", fn);
  LMOE_REQUIRE(rows >= 0 && cols > 0 && cols % 256 == 0, LMOE_ESHAPE, "%s: row length %d is not a multiple of 256", fn,
               cols);
  const long long nb = rows * (cols / 256);
  if (nb == 0) return 0;
  LMOE_REQUIRE(w && out, LMOE_EINVAL, "%s: null pointer", fn);
  hipLaunchKernelGGL(k_quantize_q4_k, dim3(unsigned((nb + 255) / 256)), dim3(256), 0, (hipStream_t)stream, w, wdtype,
                     nb, out);
  LMOE_LAUNCHED(fn);
  return 0;
}
