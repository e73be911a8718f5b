// Decode chain: gate/up + SwiGLU, and down + weighted combine, reading GGUF Q4_0 / Q4_K blocks in place.
//
// The reference runs these as gguf_gate_up / gguf_down (gguf_experts.py:452-526): LPR lanes a row, 16-bit loads
// of each 18-byte block, shuffle-tree reductions. Here, for CDNA4:
//   * each wavefront takes a task of 4 consecutive rows of one expert matrix (gate and up together), which is one
//     contiguous byte range of 144 * P bytes (P = row length / 64). Its 16-byte loads are issued first, into
//     registers, so the HBM round trip overlaps the staging of the activations; they land in the wavefront's own
//     LDS region and are read back as 36-byte "units" (64 weights: two Q4_0 blocks or a quarter Q4_K
//     super-block), each lane a unit, 9 dword reads at a 9-dword lane stride (bank-conflict free);
//   * activations are fetched with 16-byte loads into LDS, then rearranged there into f16 pairs in nibble order;
//     each unit's nibbles meet them in v_dot2_f32_f16 (lmoe_common.h), fp32 accumulation;
//   * per-unit partial sums go to LDS and are added in a fixed order (deterministic results);
//   * down adds the k experts of a token, weighted by the router scores, plus the shared expert and a residual,
//     in the same kernel, so no [T * k, H] intermediate is written.
#include <algorithm>

#include "lmoe_common.h"

namespace lmoe {

constexpr int XS = 36;  // dwords an x unit takes in LDS: 32 pairs + 4 pad (keeps lanes on distinct banks)
constexpr int RB = 4;   // rows a wavefront task covers, of each matrix

__device__ __forceinline__ int elt_size(int dt) { return dt == LMOE_F32 ? 4 : 2; }

// nbytes (a multiple of 16) from global src to LDS dst, 16 bytes a thread a step.
__device__ __forceinline__ void copy_to_lds(const void *src, void *dst, int nbytes, int tid, int nthr) {
  const u32x4 *s = static_cast<const u32x4 *>(src);
  u32x4 *d = static_cast<u32x4 *>(dst);
  for (int i = tid; i < nbytes / 16; i += nthr) d[i] = s[i];
}

__device__ __forceinline__ float lds_elt(const void *raw, int i, int dt) {
  if (dt == LMOE_F32) return static_cast<const float *>(raw)[i];
  const uint16_t b = static_cast<const uint16_t *>(raw)[i];
  return dt == LMOE_F16 ? float(__builtin_bit_cast(_Float16, b)) : bf16_to_f32(b);
}

// An activation row staged raw in LDS (64 P elements of dtype dt) -> f16 pairs in block type TQ's nibble order,
// and the sums of each 32-weight half-unit over the f16-rounded values (8 lanes a half-unit, fixed order).
template <int TQ>
__device__ __forceinline__ void permute_x(const void *raw, int dt, int P, uint32_t *xs, float *sums, int tid,
                                          int nthr) {
  constexpr int H = TQ == LMOE_Q4_K ? 32 : 16;
  for (int idx = tid; idx < 32 * P; idx += nthr) {
    const int p = idx >> 5, dw = idx & 31;
    const h2_t v = {_Float16(lds_elt(raw, 64 * p + xelem(dw, 0, H), dt)),
                    _Float16(lds_elt(raw, 64 * p + xelem(dw, 1, H), dt))};
    xs[p * XS + dw] = __builtin_bit_cast(uint32_t, v);
  }
  if (!sums) return;
  for (int base = 0; base < 16 * P; base += nthr) {
    const int idx = base + tid, hu = idx >> 3, part = idx & 7;
    float s = 0.0f;
    if (idx < 16 * P) {
#pragma unroll
      for (int i = 0; i < 4; ++i) s += float(_Float16(lds_elt(raw, 32 * hu + 4 * part + i, dt)));
    }
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    s += __shfl_xor(s, 4, 64);
    if (idx < 16 * P && part == 0) sums[hu] = s;
  }
}

__device__ __forceinline__ void load_x32(const uint32_t *xs, uint32_t *xv) {
  const u32x4 *q = reinterpret_cast<const u32x4 *>(xs);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const u32x4 v = q[i];
    xv[4 * i] = v.x;
    xv[4 * i + 1] = v.y;
    xv[4 * i + 2] = v.z;
    xv[4 * i + 3] = v.w;
  }
}

// The dot of unit p of a staged row (9 P dwords) with x pairs xv.
template <int TQ>
__device__ __forceinline__ float row_unit_dot(const uint32_t *row, int p, const uint32_t *xv, float sx0, float sx1) {
  if (TQ == LMOE_Q4_0) {
    uint32_t u[9];
#pragma unroll
    for (int i = 0; i < 9; ++i) u[i] = row[9 * p + i];
    return unit_dot_q4_0(u, xv, sx0, sx1);
  } else {
    const uint32_t *sb = row + 36 * (p >> 2);
    const int c = p & 3;
    uint32_t hdr[4], q[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) hdr[i] = sb[i];
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = sb[4 + 8 * c + i];
    return unit_dot_q4_k(hdr, q, c, xv, sx0, sx1);
  }
}

// ---- gate/up --------------------------------------------------------------------------------------------------
//
// Grid (I / (4 NW), n_slots), NW wavefronts a workgroup; wavefront w of block (bx, s) takes rows
// [(bx NW + w) 4, +4) of gate and up of expert slots[s]; NC >= ceil(9 P / 64) 16-byte chunks a lane a matrix.
// LDS: x pairs for TG (and TU when it differs), the half-unit sums, then a region that first holds the raw x row
// and then each wavefront's 8 staged rows, then each wavefront's 8 x (P + 1) partial sums.
template <int TG, int TU, int NC, int NW>
__global__ void __launch_bounds__(64 * NW)
    k_gate_up(const void *x, int xdt, const uint32_t *slots, int topk, const uint8_t *wg, const uint8_t *wu,
              int n_experts, int I, float *h, int P) {
  constexpr bool SAME = TG == TU;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int s = blockIdx.y;
  const uint32_t e = slots[s];
  const int r0 = (blockIdx.x * NW + wave) * RB;
  if (e >= uint32_t(n_experts)) {  // no such expert: zero rows (cpu_kern.cpp:316-318)
    if (lane < RB && r0 + lane < I) h[size_t(s) * I + r0 + lane] = 0.0f;
    return;
  }
  extern __shared__ u32x4 lds4[];
  uint32_t *xg = reinterpret_cast<uint32_t *>(lds4);
  uint32_t *xu = SAME ? xg : xg + P * XS;
  float *sums = reinterpret_cast<float *>(xu + P * XS);
  const int sum_sz = (2 * P + 3) & ~3;
  uint32_t *region = reinterpret_cast<uint32_t *>(sums + sum_sz);
  const int stage_dw = 2 * RB * 9 * P;
  const int xraw_dw = 16 * P * elt_size(xdt);  // 64 P elements
  uint32_t *stage = region + wave * stage_dw;
  float *red = reinterpret_cast<float *>(region + max(NW * stage_dw, xraw_dw)) + wave * (2 * RB * (P + 1));

  // 1) this wavefront's 8 rows, 9 P 16-byte chunks a matrix, into registers
  const int C = 9 * P;
  const bool rows_ok = r0 < I;
  const size_t rowb = size_t(36) * P;
  const u32x4 *gsrc = reinterpret_cast<const u32x4 *>(wg + (size_t(e) * I + r0) * rowb);
  const u32x4 *usrc = reinterpret_cast<const u32x4 *>(wu + (size_t(e) * I + r0) * rowb);
  u32x4 vg[NC], vu[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = lane + 64 * i;
    if (rows_ok && c < C) {
      vg[i] = __builtin_nontemporal_load(gsrc + c);
      vu[i] = __builtin_nontemporal_load(usrc + c);
    }
  }
  // 2) the x row, raw, then rearranged
  const int xbytes = 64 * P * elt_size(xdt);
  copy_to_lds(static_cast<const char *>(x) + size_t(s / topk) * xbytes, region, xbytes, threadIdx.x, 64 * NW);
  __syncthreads();
  permute_x<TG>(region, xdt, P, xg, sums, threadIdx.x, 64 * NW);
  if (!SAME) permute_x<TU>(region, xdt, P, xu, nullptr, threadIdx.x, 64 * NW);
  __syncthreads();
  if (!rows_ok) return;
  u32x4 *st4 = reinterpret_cast<u32x4 *>(stage);
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = lane + 64 * i;
    if (c < C) {
      st4[c] = vg[i];
      st4[C + c] = vu[i];
    }
  }
  __builtin_amdgcn_wave_barrier();

  const int U = 2 * RB * P;
  if (SAME && (64 % P) == 0) {  // each lane keeps one unit column: its x pairs load once
    const int p = lane % P;
    uint32_t xv[32];
    load_x32(xg + p * XS, xv);
    const float sx0 = sums[2 * p], sx1 = sums[2 * p + 1];
    for (int u = lane; u < U; u += 64) {
      const int row = u / P;
      red[row * (P + 1) + p] = row_unit_dot<TG>(stage + row * 9 * P, p, xv, sx0, sx1);
    }
  } else {
    for (int u = lane; u < U; u += 64) {
      const int row = u / P, p = u - row * P;
      uint32_t xv[32];
      const float sx0 = sums[2 * p], sx1 = sums[2 * p + 1];
      float part;
      if (row < RB) {
        load_x32(xg + p * XS, xv);
        part = row_unit_dot<TG>(stage + row * 9 * P, p, xv, sx0, sx1);
      } else {
        load_x32(xu + p * XS, xv);
        part = row_unit_dot<TU>(stage + row * 9 * P, p, xv, sx0, sx1);
      }
      red[row * (P + 1) + p] = part;
    }
  }
  __builtin_amdgcn_wave_barrier();

  // 8 rows x P partials: 8 lanes a row, fixed order
  constexpr int LPR = 64 / (2 * RB);
  const int rr = lane / LPR, sub = lane % LPR;
  float acc = 0.0f;
  for (int p = sub; p < P; p += LPR) acc += red[rr * (P + 1) + p];
#pragma unroll
  for (int m = LPR / 2; m > 0; m >>= 1) acc += __shfl_xor(acc, m, 64);
  const float up = __shfl_xor(acc, RB * LPR, 64);  // up row rr sits RB * LPR = 32 lanes above gate row rr
  if (rr < RB && sub == 0 && r0 + rr < I) h[size_t(s) * I + r0 + rr] = silu_mul(acc, up);
}

// ---- down + combine -------------------------------------------------------------------------------------------
//
// Grid (H / (4 NW), T). Block (bx, t) stages h rows t k .. t k + k - 1 as x pairs, then wavefront w takes output
// rows [(bx NW + w) 4, +4) of all k experts of token t, adds them weighted by scores[t] (1 when scores is null),
// then the gated shared-expert row and the residual, and writes out[t]. When k 9 P <= 64 NC the weight chunks are
// fetched into registers before the h staging; otherwise after it.
template <int TD, int NC, int NW>
__global__ void __launch_bounds__(64 * NW)
    k_down_combine(const float *h, const uint32_t *ids, const float *scores, int k, const uint8_t *wd,
                   int n_experts, int I, int H, const float *shared, const float *gate, int gate_stride,
                   const void *residual, int rdt, void *out, int odt) {
  const int P = I / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = blockIdx.y;
  const int n0 = (blockIdx.x * NW + wave) * RB;
  extern __shared__ u32x4 lds4[];
  const int sum_sz = (2 * P + 3) & ~3;
  uint32_t *hx = reinterpret_cast<uint32_t *>(lds4);                // k * P * XS
  float *hs = reinterpret_cast<float *>(hx + k * P * XS);            // k * sum_sz
  uint32_t *eid = reinterpret_cast<uint32_t *>(hs + k * sum_sz);    // 32
  float *esc = reinterpret_cast<float *>(eid + 32);                 // 32
  uint32_t *region = reinterpret_cast<uint32_t *>(esc + 32);
  const int stage_dw = k * RB * 9 * P;
  uint32_t *stage = region + wave * stage_dw;
  const int red_ld = k * P + 1;
  float *red = reinterpret_cast<float *>(region + max(NW * stage_dw, k * I)) + wave * (RB * red_ld);

  const size_t rowb = size_t(36) * P;
  const int C = 9 * P;  // 16-byte chunks of 4 rows
  const bool rows_ok = n0 < H;
  const bool pre = k * C <= 64 * NC;
  const uint32_t *tid_ids = ids + size_t(t) * k;
  u32x4 v[NC];
  if (pre && rows_ok) {
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = lane + 64 * i;
      if (c < k * C) {
        const int j = c / C, cc = c - j * C;
        const uint32_t e = tid_ids[j];
        if (e < uint32_t(n_experts))
          v[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(wd + (size_t(e) * H + n0) * rowb) + cc);
      }
    }
  }
  copy_to_lds(h + size_t(t) * k * I, region, k * I * 4, threadIdx.x, 64 * NW);
  if (threadIdx.x < k) {
    eid[threadIdx.x] = tid_ids[threadIdx.x];
    esc[threadIdx.x] = scores ? scores[size_t(t) * k + threadIdx.x] : 1.0f;
  }
  __syncthreads();
  for (int j = 0; j < k; ++j)
    permute_x<TD>(region + j * I, LMOE_F32, P, hx + j * P * XS, hs + j * sum_sz, threadIdx.x, 64 * NW);
  __syncthreads();
  if (!rows_ok) return;

  u32x4 *st4 = reinterpret_cast<u32x4 *>(stage);
  if (pre) {
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = lane + 64 * i;
      if (c < k * C && eid[c / C] < uint32_t(n_experts)) st4[c] = v[i];
    }
  } else {
    for (int j = 0; j < k; ++j) {
      const uint32_t e = eid[j];
      if (e >= uint32_t(n_experts)) continue;
      const u32x4 *src = reinterpret_cast<const u32x4 *>(wd + (size_t(e) * H + n0) * rowb);
      for (int c = lane; c < C; c += 64) st4[j * C + c] = __builtin_nontemporal_load(src + c);
    }
  }
  __builtin_amdgcn_wave_barrier();

  const int U = k * RB * P;
  for (int u = lane; u < U; u += 64) {
    const int j = u / (RB * P), rem = u - j * (RB * P), row = rem / P, p = rem - row * P;
    float part = 0.0f;
    if (eid[j] < uint32_t(n_experts)) {
      uint32_t xv[32];
      load_x32(hx + (j * P + p) * XS, xv);
      const float *sj = hs + j * sum_sz;
      part = esc[j] * row_unit_dot<TD>(stage + (j * RB + row) * 9 * P, p, xv, sj[2 * p], sj[2 * p + 1]);
    }
    red[row * red_ld + j * P + p] = part;
  }
  __builtin_amdgcn_wave_barrier();

  constexpr int LPR = 64 / RB;
  const int rr = lane / LPR, sub = lane % LPR;
  float acc = 0.0f;
  for (int i = sub; i < k * P; i += LPR) acc += red[rr * red_ld + i];
#pragma unroll
  for (int m = LPR / 2; m > 0; m >>= 1) acc += __shfl_xor(acc, m, 64);
  const int n = n0 + rr;
  if (sub == 0 && n < H) {
    const size_t o = size_t(t) * H + n;
    if (shared) acc += sigmoidf_(gate[size_t(t) * gate_stride]) * shared[o];
    if (residual) acc += load_elt(residual, o, rdt);
    store_elt(out, o, acc, odt);
  }
}

// ---- host dispatch ----------------------------------------------------------------------------------------------

template <int TG, int TU, int NC, int NW>
static int launch_gate_up(const void *x, int xdt, const uint32_t *slots, int n_slots, int topk, const uint8_t *wg,
                          const uint8_t *wu, int n_experts, int H, int I, float *h, hipStream_t st) {
  const int P = H / 64;
  const int sum_sz = (2 * P + 3) & ~3;
  const size_t stage_dw = size_t(2) * RB * 9 * P, xraw_dw = size_t(16) * P * (xdt == LMOE_F32 ? 4 : 2);
  const size_t lds = size_t(4) * ((TG == TU ? 1 : 2) * P * XS + sum_sz + std::max(NW * stage_dw, xraw_dw) +
                                  NW * 2 * RB * (P + 1));
  LMOE_REQUIRE(lds <= 160 * 1024, LMOE_ESHAPE, "lmoe_gemv_gate_up: hidden %d needs %zu bytes of LDS", H, lds);
  const dim3 grid((I + RB * NW - 1) / (RB * NW), n_slots);
  if (int rc = allow_lds(k_gate_up<TG, TU, NC, NW>, lds, "lmoe_gemv_gate_up")) return rc;
  hipLaunchKernelGGL((k_gate_up<TG, TU, NC, NW>), grid, dim3(64 * NW), lds, st, x, xdt, slots, topk, wg, wu,
                     n_experts, I, h, P);
  LMOE_LAUNCHED("lmoe_gemv_gate_up");
  return 0;
}

template <int TG, int TU>
static int gate_up_p(const void *x, int xdt, const uint32_t *slots, int n_slots, int topk, const uint8_t *wg,
                     const uint8_t *wu, int n_experts, int H, int I, float *h, hipStream_t st) {
  const int nc = (9 * (H / 64) + 63) / 64;  // 16-byte chunks a lane a matrix
  if (nc <= 2) return launch_gate_up<TG, TU, 2, 4>(x, xdt, slots, n_slots, topk, wg, wu, n_experts, H, I, h, st);
  if (nc <= 4) return launch_gate_up<TG, TU, 4, 4>(x, xdt, slots, n_slots, topk, wg, wu, n_experts, H, I, h, st);
  if (nc <= 6) return launch_gate_up<TG, TU, 6, 4>(x, xdt, slots, n_slots, topk, wg, wu, n_experts, H, I, h, st);
  if (nc <= 9) return launch_gate_up<TG, TU, 9, 2>(x, xdt, slots, n_slots, topk, wg, wu, n_experts, H, I, h, st);
  if (nc <= 12) return launch_gate_up<TG, TU, 12, 2>(x, xdt, slots, n_slots, topk, wg, wu, n_experts, H, I, h, st);
  return fail(LMOE_ESHAPE, "lmoe_gemv_gate_up: hidden %d is above the 5376 this kernel stages", H);
}

static int check_matrix(const char *fn, int type, int rows, int cols, const void *buf) {
  LMOE_REQUIRE(qtype_ok(type), LMOE_ETYPE, "%s: ggml type %d is not supported (Q4_0 = 2, Q4_K = 12)", fn, type);
  LMOE_REQUIRE(cols > 0 && cols % block_weights(type) == 0 && cols % 64 == 0, LMOE_ESHAPE,
               "%s: row length %d is not a multiple of %d", fn, cols, type == LMOE_Q4_K ? 256 : 64);
  LMOE_REQUIRE(rows > 0 && rows % 4 == 0, LMOE_ESHAPE, "%s: %d rows is not a multiple of 4", fn, rows);
  LMOE_REQUIRE(buf && aligned16(buf), LMOE_EALIGN, "%s: expert buffer must be 16-byte aligned", fn);
  return 0;
}

}  // namespace lmoe

using namespace lmoe;

extern "C" int lmoe_gemv_gate_up(const void *x, int xdtype, const uint32_t *slots, int n_slots, int topk,
                                 const uint8_t *wg, const uint8_t *wu, int type_g, int type_u, int n_experts, int H,
                                 int I, float *h, void *stream) {
  const char *fn = "lmoe_gemv_gate_up";
  LMOE_REQUIRE(dtype_ok(xdtype), LMOE_EINVAL, "%s: x dtype %d is not F32, F16 or BF16", fn, xdtype);
  LMOE_REQUIRE(n_slots >= 0 && topk > 0 && n_slots % topk == 0, LMOE_ESHAPE,
               "%s: %d slots is not a multiple of topk %d", fn, n_slots, topk);
  LMOE_REQUIRE(n_experts > 0, LMOE_ESHAPE, "%s: no experts", fn);
  if (int rc = check_matrix(fn, type_g, I, H, wg)) return rc;
  if (int rc = check_matrix(fn, type_u, I, H, wu)) return rc;
  if (n_slots == 0) return 0;
  LMOE_REQUIRE(x && slots && h, LMOE_EINVAL, "%s: null pointer", fn);
  LMOE_REQUIRE(aligned16(x), LMOE_EALIGN, "%s: x must be 16-byte aligned", fn);
  hipStream_t st = (hipStream_t)stream;
  if (type_g == LMOE_Q4_0 && type_u == LMOE_Q4_0)
    return gate_up_p<LMOE_Q4_0, LMOE_Q4_0>(x, xdtype, slots, n_slots, topk, wg, wu, n_experts, H, I, h, st);
  if (type_g == LMOE_Q4_K && type_u == LMOE_Q4_K)
    return gate_up_p<LMOE_Q4_K, LMOE_Q4_K>(x, xdtype, slots, n_slots, topk, wg, wu, n_experts, H, I, h, st);
  if (type_g == LMOE_Q4_0)
    return gate_up_p<LMOE_Q4_0, LMOE_Q4_K>(x, xdtype, slots, n_slots, topk, wg, wu, n_experts, H, I, h, st);
  return gate_up_p<LMOE_Q4_K, LMOE_Q4_0>(x, xdtype, slots, n_slots, topk, wg, wu, n_experts, H, I, h, st);
}

extern "C" int lmoe_gemv_down_combine(const float *h, const uint32_t *ids, const float *scores, int T, int k,
                                      const uint8_t *wd, int type_d, int n_experts, int I, int H, const float *shared,
                                      const float *gate, int gate_stride, const void *residual, int rdtype,
                                      void *out, int odtype, void *stream) {
  const char *fn = "lmoe_gemv_down_combine";
  LMOE_REQUIRE(dtype_ok(odtype) && (!residual || dtype_ok(rdtype)), LMOE_EINVAL, "%s: bad dtype", fn);
  LMOE_REQUIRE(T >= 0 && k > 0 && k <= 32, LMOE_ESHAPE, "%s: k %d is outside 1..32", fn, k);
  LMOE_REQUIRE(n_experts > 0, LMOE_ESHAPE, "%s: no experts", fn);
  LMOE_REQUIRE(!shared == !gate, LMOE_EINVAL, "%s: shared and gate go together", fn);
  if (int rc = check_matrix(fn, type_d, H, I, wd)) return rc;
  if (T == 0) return 0;
  LMOE_REQUIRE(h && ids && out, LMOE_EINVAL, "%s: null pointer", fn);
  LMOE_REQUIRE(aligned16(h), LMOE_EALIGN, "%s: h must be 16-byte aligned", fn);
  constexpr int NW = 2, NC = 16;
  const int P = I / 64;
  const int sum_sz = (2 * P + 3) & ~3;
  const size_t stage_dw = size_t(k) * RB * 9 * P;
  const size_t lds = size_t(4) * (k * P * XS + k * sum_sz + 64 + std::max(NW * stage_dw, size_t(k) * I) +
                                  NW * RB * (k * P + 1));
  LMOE_REQUIRE(lds <= 160 * 1024, LMOE_ESHAPE, "%s: k %d at width %d needs %zu bytes of LDS", fn, k, I, lds);
  const dim3 grid((H + RB * NW - 1) / (RB * NW), T);
  hipStream_t st = (hipStream_t)stream;
  if (type_d == LMOE_Q4_0) {
    if (int rc = allow_lds(k_down_combine<LMOE_Q4_0, NC, NW>, lds, fn)) return rc;
    hipLaunchKernelGGL((k_down_combine<LMOE_Q4_0, NC, NW>), grid, dim3(64 * NW), lds, st, h, ids, scores, k, wd,
                       n_experts, I, H, shared, gate, gate_stride, residual, rdtype, out, odtype);
  } else {
    if (int rc = allow_lds(k_down_combine<LMOE_Q4_K, NC, NW>, lds, fn)) return rc;
    hipLaunchKernelGGL((k_down_combine<LMOE_Q4_K, NC, NW>), grid, dim3(64 * NW), lds, st, h, ids, scores, k, wd,
                       n_experts, I, H, shared, gate, gate_stride, residual, rdtype, out, odtype);
  }
  LMOE_LAUNCHED(fn);
  return 0;
}
