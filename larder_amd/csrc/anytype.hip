// The ggml block types beyond Q4_0 / Q4_K: Q4_1, Q5_K, Q6_K and Q8_0, on the decode chain and in dequant.
//
// The reference decodes all of them with one task function per type (gguf_experts.py:78-373: gg_task / gg_task8
// hand a kernel 8 or 32 weights of a row at a time) inside the same GATE_UP / DOWN kernels. Here the Q4 pair keeps
// its specialised kernels (36-byte units, prepared activations, v_dot2 on nibbles); every type, Q4 included, also
// has a 32-weight decoder below, and two general GEMV kernels run on it whenever a projection's type is not a Q4
// one: one lane a 32-weight chunk of a row, x (or the token's h rows) staged in LDS as float32, one runtime type
// switch a row outside the chunk loop. Mixed layers work: gate/up in Q4_K on the specialised kernel, down in Q6_K
// here (the 35B UD-Q4_K_XL mix), with h passed as float32.
//
// Dequant follows ggml's arithmetic with every multiply and add rounded on its own (the library builds with
// -ffp-contract=off), so lmoe_dequant is bit-exact with the CPU restatement for every type:
//   Q4_0 (q - 8) d             Q4_1 q d + m               Q8_0 q d
//   Q4_K (d sc) q - (dmin m)   Q5_K the same, q += 16 bit  Q6_K (d sc) (q - 32)
// Block layouts (ggml, gguf_ref.py:253-276, 345-355, 392-401): Q4_1 = f16 d, f16 m, 16 qs bytes (weight j low
// nibble of byte j, j + 16 high); Q8_0 = f16 d, 32 int8; Q5_K = f16 d, f16 dmin, 12 scale bytes, qh[32], qs[128];
// Q6_K = ql[128], qh[64], int8 sc[16], f16 d.
#include "lmoe_common.h"

namespace lmoe {

bool qtype_any(int t) {
  return t == LMOE_Q4_0 || t == LMOE_Q4_K || t == LMOE_Q4_1 || t == LMOE_Q5_K || t == LMOE_Q6_K || t == LMOE_Q8_0;
}
int block_weights_any(int t) { return (t == LMOE_Q4_K || t == LMOE_Q5_K || t == LMOE_Q6_K) ? 256 : 32; }
int block_bytes_any(int t) {
  switch (t) {
    case LMOE_Q4_0: return 18;
    case LMOE_Q4_1: return 20;
    case LMOE_Q8_0: return 34;
    case LMOE_Q4_K: return 144;
    case LMOE_Q5_K: return 176;
    case LMOE_Q6_K: return 210;
  }
  return 0;
}
// the alignment every block of the type keeps when the buffer starts 16-byte aligned
static int block_align(int t) { return (t == LMOE_Q4_K || t == LMOE_Q5_K) ? 16 : t == LMOE_Q4_1 ? 4 : 2; }

// 2-byte aligned reads (every block of every type is at least 2-byte aligned)
__device__ __forceinline__ uint32_t ld16(const uint8_t *p) { return *reinterpret_cast<const uint16_t *>(p); }
__device__ __forceinline__ uint32_t ld32h(const uint8_t *p) { return ld16(p) | (ld16(p + 2) << 16); }
__device__ __forceinline__ uint32_t ld32(const uint8_t *p) { return *reinterpret_cast<const uint32_t *>(p); }
__device__ __forceinline__ float f16at(const uint8_t *p) { return float(__builtin_bit_cast(_Float16, uint16_t(ld16(p)))); }

// 32 bytes at a 2-byte aligned address as 8 dwords: the 9 dwords from the 4-byte aligned address at or below it
// (two 16-byte loads, which need only dword alignment, and a dword), realigned by the address's low 2 bits. The
// window reaches 2 bytes below p when p is 2 mod 4 (never the start of an allocation) and up to p + 36: callers keep
// p + 36 inside the block.
typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
__device__ __forceinline__ void load_window8(const uint8_t *p, uint32_t (&o)[8]) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  const uint32_t *base = reinterpret_cast<const uint32_t *>(a & ~uintptr_t(3));
  const u32x4a4 v0 = *reinterpret_cast<const u32x4a4 *>(base), v1 = *reinterpret_cast<const u32x4a4 *>(base + 4);
  const uint32_t v8 = base[8];
  const uint32_t w[9] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w, v8};
  const uint32_t sh = uint32_t(a & 3);
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], sh);
}

// The 32 weights of chunk c (weights 32 c .. 32 c + 31) of a row of type T, in natural order.
template <int T>
__device__ __forceinline__ void decode32(const uint8_t *row, int c, float *w) {
  if (T == LMOE_Q4_0 || T == LMOE_Q4_1) {
    const uint8_t *b = row + size_t(c) * (T == LMOE_Q4_0 ? 18 : 20);
    const float d = f16at(b);
    const float m = T == LMOE_Q4_1 ? f16at(b + 2) : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t q = T == LMOE_Q4_0 ? ld32h(b + 2 + 4 * i) : ld32(b + 4 + 4 * i);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int lo = int((q >> (8 * j)) & 15u), hi = int((q >> (8 * j + 4)) & 15u);
        if (T == LMOE_Q4_0) {
          w[4 * i + j] = float(lo - 8) * d;
          w[16 + 4 * i + j] = float(hi - 8) * d;
        } else {
          w[4 * i + j] = float(lo) * d + m;
          w[16 + 4 * i + j] = float(hi) * d + m;
        }
      }
    }
  } else if (T == LMOE_Q8_0) {
    const uint8_t *b = row + size_t(c) * 34;
    const float d = f16at(b);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t q = ld32h(b + 2 + 4 * i);
#pragma unroll
      for (int j = 0; j < 4; ++j) w[4 * i + j] = float(int(int8_t(uint8_t(q >> (8 * j))))) * d;
    }
  } else if (T == LMOE_Q4_K || T == LMOE_Q5_K) {
    const uint8_t *b = row + size_t(c >> 3) * (T == LMOE_Q4_K ? 144 : 176);
    const int j = c & 7;
    const uint32_t h0 = ld32(b), s0 = ld32(b + 4), s1 = ld32(b + 8), s2 = ld32(b + 12);
    float sc, mn;
    k4_scale_min(s0, s1, s2, j, &sc, &mn);
    const float d1 = half_lo(h0) * sc, m1 = half_hi(h0) * mn;
    const uint8_t *qs = b + (T == LMOE_Q4_K ? 16 : 48) + 32 * (j >> 1);
    const int sh = 4 * (j & 1);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t q = ld32(qs + 4 * i);
      const uint32_t qh = T == LMOE_Q5_K ? ld32(b + 16 + 4 * i) : 0u;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        int v = int((q >> (8 * k + sh)) & 15u);
        if (T == LMOE_Q5_K) v += 16 * int((qh >> (8 * k + j)) & 1u);
        w[4 * i + k] = d1 * float(v) - m1;
      }
    }
  } else {  // Q6_K: chunk j = 4 h + g of the super-block
    const uint8_t *b = row + size_t(c >> 3) * 210;
    const int j = c & 7, h = j >> 2, g = j & 3;
    // the super-block is 2-byte aligned: its 32 ql and 32 qh bytes come as 9-dword windows from the 4-byte
    // aligned address below them (two 16-byte loads and one dword each, instead of 16 halfword pairs; the windows
    // end by byte 196 of the 210) and are realigned by the 0 or 2 byte offset
    uint32_t lq[8], hq[8];
    load_window8(b + 64 * h + 32 * (g & 1), lq);
    load_window8(b + 128 + 32 * h, hq);
    const float d = f16at(b + 208);
    const uint32_t scw = ld16(b + 192 + 8 * h + 2 * g);
    const float ds0 = d * float(int(int8_t(uint8_t(scw)))), ds1 = d * float(int(int8_t(uint8_t(scw >> 8))));
    const int sl = 4 * (g >> 1), shh = 2 * g;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t lw = lq[i], hw = hq[i];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int v = int(((lw >> (8 * k + sl)) & 15u) | (((hw >> (8 * k + shh)) & 3u) << 4)) - 32;
        w[4 * i + k] = (i < 4 ? ds0 : ds1) * float(v);
      }
    }
  }
}

template <int T>
__device__ __forceinline__ float chunks_dot(const uint8_t *row, int n_chunks, const float *xs, int lane) {
  float acc = 0.0f;
  for (int c = lane; c < n_chunks; c += 64) {
    float w[32];
    decode32<T>(row, c, w);
    const float4 *xv = reinterpret_cast<const float4 *>(xs + 32 * c);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 v = xv[i];
      acc = fmaf(w[4 * i], v.x, acc);
      acc = fmaf(w[4 * i + 1], v.y, acc);
      acc = fmaf(w[4 * i + 2], v.z, acc);
      acc = fmaf(w[4 * i + 3], v.w, acc);
    }
  }
  return acc;
}

// This lane's part of row . x over the row's n_chunks 32-weight chunks (chunk lane, lane + 64, ...); type is
// uniform across the wavefront.
__device__ __forceinline__ float row_dot_any(const uint8_t *row, int type, int n_chunks, const float *xs, int lane) {
  switch (type) {
    case LMOE_Q4_0: return chunks_dot<LMOE_Q4_0>(row, n_chunks, xs, lane);
    case LMOE_Q4_1: return chunks_dot<LMOE_Q4_1>(row, n_chunks, xs, lane);
    case LMOE_Q8_0: return chunks_dot<LMOE_Q8_0>(row, n_chunks, xs, lane);
    case LMOE_Q4_K: return chunks_dot<LMOE_Q4_K>(row, n_chunks, xs, lane);
    case LMOE_Q5_K: return chunks_dot<LMOE_Q5_K>(row, n_chunks, xs, lane);
    default: return chunks_dot<LMOE_Q6_K>(row, n_chunks, xs, lane);
  }
}

constexpr int kAnyRows = 2;  // rows a wavefront, 4 wavefronts a workgroup

// The partial dots of a wavefront's rows r0, r0 + 1 of gate and up (both type T), every load issued before any
// sum: one 32-weight chunk a lane a row (H <= 2048; wider rows loop).
template <int T>
__device__ __forceinline__ void gate_up_rows(const uint8_t *wg, const uint8_t *wu, size_t rb, int H, const float *xs,
                                             int lane, float *pg, float *pu) {
#pragma unroll
  for (int rr = 0; rr < kAnyRows; ++rr) {
    pg[rr] = chunks_dot<T>(wg + rr * rb, H / 32, xs, lane);
    pu[rr] = chunks_dot<T>(wu + rr * rb, H / 32, xs, lane);
  }
}

// Grid (ceil(I / 8), n_slots), 256 threads: slot s's x row (s / topk) staged as float32 in LDS; wavefront w takes
// rows 8 bx + 2 w, +1 of the slot's expert, gate and up, and writes h[s][r] = silu(g) u (float32). A slot past the
// experts gives zeros (cpu_kern.cpp:316-318). Rows past I (I odd in pairs) repeat the last row and are not stored.
__global__ void __launch_bounds__(256) k_gate_up_any(const void *x, int xdt, const uint32_t *slots, int topk,
                                                     const uint8_t *wg, const uint8_t *wu, int tg, int tu,
                                                     int n_experts, int H, int I, size_t rbg, size_t rbu, float *h) {
  extern __shared__ float xs[];
  const int s = blockIdx.y;
  const uint32_t e = slots[s];
  const size_t xr = size_t(s / topk) * H;
  for (int i = threadIdx.x; i < H; i += 256) xs[i] = load_elt(x, xr + i, xdt);
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r0 = (blockIdx.x * 4 + wave) * kAnyRows;
  if (r0 >= I) return;
  const bool ok = e < uint32_t(n_experts);
  const int rb0 = min(r0, I - kAnyRows);  // I is even: both rows in range
  const uint32_t ee = ok ? e : 0u;
  const uint8_t *pgw = wg + (size_t(ee) * I + rb0) * rbg, *puw = wu + (size_t(ee) * I + rb0) * rbu;
  float pg[kAnyRows], pu[kAnyRows];
  if (tg == tu) {
    switch (tg) {
      case LMOE_Q4_0: gate_up_rows<LMOE_Q4_0>(pgw, puw, rbg, H, xs, lane, pg, pu); break;
      case LMOE_Q4_1: gate_up_rows<LMOE_Q4_1>(pgw, puw, rbg, H, xs, lane, pg, pu); break;
      case LMOE_Q8_0: gate_up_rows<LMOE_Q8_0>(pgw, puw, rbg, H, xs, lane, pg, pu); break;
      case LMOE_Q4_K: gate_up_rows<LMOE_Q4_K>(pgw, puw, rbg, H, xs, lane, pg, pu); break;
      case LMOE_Q5_K: gate_up_rows<LMOE_Q5_K>(pgw, puw, rbg, H, xs, lane, pg, pu); break;
      default: gate_up_rows<LMOE_Q6_K>(pgw, puw, rbg, H, xs, lane, pg, pu); break;
    }
  } else {
#pragma unroll
    for (int rr = 0; rr < kAnyRows; ++rr) {
      pg[rr] = row_dot_any(pgw + rr * rbg, tg, H / 32, xs, lane);
      pu[rr] = row_dot_any(puw + rr * rbu, tu, H / 32, xs, lane);
    }
  }
#pragma unroll
  for (int rr = 0; rr < kAnyRows; ++rr) {
    const float g = wave_sum(pg[rr]), u = wave_sum(pu[rr]);
    const int r = rb0 + rr;
    if (lane == 0 && r >= r0) h[size_t(s) * I + r] = ok ? silu_mul(g, u) : 0.0f;
  }
}

// One token's weighted sum over its k experts of rows o0, o0 + 1 of down (type T), every expert's loads issued
// before the sums: acc[rr] = sum_j s_j (h_j . wd[e_j][o0 + rr]) as this lane's part.
// The token's k experts x I / 32 chunks are one list of (expert j, chunk c) items, item u = j (I / 32) + c; lane
// takes u = lane, lane + 64, ... two a pass, so that at decode width (k 8, I 768: 192 items) every lane has work and
// both items' loads are out before either's arithmetic (a loop over the experts kept 40 of 64 lanes idle at I 768
// and paid one memory round trip an expert). A lane's clamped repeat of the last item takes weight 0. FLAT = false,
// for rows of at most 64 items (the decode chain's one slot a row, k 1), keeps that loop: it needs neither the second
// item's registers nor its pass.
template <int T, bool FLAT>
__device__ __forceinline__ void down_rows(const uint8_t *wd, size_t rb, int H, int I, int k, int n_experts,
                                          const uint32_t *eid, const float *esc, const float *hs, int lane,
                                          float *acc) {
  if (!FLAT) {  // a row's items fit one pass (k I / 32 <= 64): chunks over lanes, one expert after another
    for (int j = 0; j < k; ++j) {
      const uint32_t e = eid[j];
      const float sc = e < uint32_t(n_experts) ? esc[j] : 0.0f;
      const uint8_t *row = wd + (size_t(e < uint32_t(n_experts) ? e : 0u) * H) * rb;
#pragma unroll
      for (int rr = 0; rr < kAnyRows; ++rr)
        acc[rr] = fmaf(sc, chunks_dot<T>(row + rr * rb, I / 32, hs + size_t(j) * I, lane), acc[rr]);
    }
    return;
  }
  const int nch = I / 32, n = k * nch;
  for (int u0 = lane; u0 - lane < n; u0 += 128) {
    // the pass's second item only when a lane of the wavefront has one (uniform: u0 - lane is); otherwise it would
    // be a whole wavefront of repeats (k 1, I 768: 24 items a row)
    const int nq = u0 - lane + 64 < n ? 2 : 1;
    float w[2][kAnyRows][32];
    float sc[2] = {0.0f, 0.0f};
    int hj[2] = {0, 0};
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      if (q >= nq) break;
      const int u = min(u0 + 64 * q, n - 1), j = u / nch, c = u - j * nch;
      const uint32_t e = eid[j];
      sc[q] = u0 + 64 * q < n && e < uint32_t(n_experts) ? esc[j] : 0.0f;
      hj[q] = j * I + 32 * c;
      const uint8_t *row = wd + (size_t(e < uint32_t(n_experts) ? e : 0u) * H) * rb;
#pragma unroll
      for (int rr = 0; rr < kAnyRows; ++rr) decode32<T>(row + rr * rb, c, w[q][rr]);
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      if (q >= nq) break;
      const float4 *xv = reinterpret_cast<const float4 *>(hs + hj[q]);
#pragma unroll
      for (int rr = 0; rr < kAnyRows; ++rr) {
        float d = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float4 v = xv[i];
          d = fmaf(w[q][rr][4 * i], v.x, d);
          d = fmaf(w[q][rr][4 * i + 1], v.y, d);
          d = fmaf(w[q][rr][4 * i + 2], v.z, d);
          d = fmaf(w[q][rr][4 * i + 3], v.w, d);
        }
        acc[rr] = fmaf(sc[q], d, acc[rr]);
      }
    }
  }
}

// Grid (ceil(H / 8), T), 256 threads: token t's k h rows staged as float32 in LDS; wavefront w takes output rows
// 8 bx + 2 w, +1: out[t][o] = sum_j s_j (h[t k + j] . wd[ids[t k + j]][o]) (+ sigmoid(gate) shared) (+ residual),
// s_j = scores[t k + j] (1 without scores), ids past the experts adding nothing (expert 0's row read, weight 0).
template <bool FLAT>
__global__ void __launch_bounds__(256)
    k_down_any(const float *h, const uint32_t *ids, const float *scores, int k, const uint8_t *wd, int td,
               int n_experts, int I, int H, size_t rbd, const float *shared, const float *gate, int gate_stride,
               const void *residual, int rdt, void *out, int odt) {
  extern __shared__ float hs[];
  __shared__ uint32_t eid[32];
  __shared__ float esc[32];
  const int t = blockIdx.y;
  for (int i = threadIdx.x; i < k * I; i += 256) hs[i] = h[size_t(t) * k * I + i];
  if (threadIdx.x < k) {
    eid[threadIdx.x] = ids[size_t(t) * k + threadIdx.x];
    esc[threadIdx.x] = scores ? scores[size_t(t) * k + threadIdx.x] : 1.0f;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int o0 = (blockIdx.x * 4 + wave) * kAnyRows;
  if (o0 >= H) return;
  const int ob = min(o0, H - kAnyRows);  // H is even: both rows in range
  const uint8_t *w0 = wd + size_t(ob) * rbd;
  float acc[kAnyRows] = {0.0f, 0.0f};
  switch (td) {
    case LMOE_Q4_0: down_rows<LMOE_Q4_0, FLAT>(w0, rbd, H, I, k, n_experts, eid, esc, hs, lane, acc); break;
    case LMOE_Q4_1: down_rows<LMOE_Q4_1, FLAT>(w0, rbd, H, I, k, n_experts, eid, esc, hs, lane, acc); break;
    case LMOE_Q8_0: down_rows<LMOE_Q8_0, FLAT>(w0, rbd, H, I, k, n_experts, eid, esc, hs, lane, acc); break;
    case LMOE_Q4_K: down_rows<LMOE_Q4_K, FLAT>(w0, rbd, H, I, k, n_experts, eid, esc, hs, lane, acc); break;
    case LMOE_Q5_K: down_rows<LMOE_Q5_K, FLAT>(w0, rbd, H, I, k, n_experts, eid, esc, hs, lane, acc); break;
    default: down_rows<LMOE_Q6_K, FLAT>(w0, rbd, H, I, k, n_experts, eid, esc, hs, lane, acc); break;
  }
#pragma unroll
  for (int rr = 0; rr < kAnyRows; ++rr) {
    float v = wave_sum(acc[rr]);
    const int o = ob + rr;
    if (lane == 0 && o >= o0) {
      const size_t oi = size_t(t) * H + o;
      if (shared) v += sigmoidf_(gate[size_t(t) * gate_stride]) * shared[oi];
      if (residual) v += load_elt(residual, oi, rdt);
      store_elt(out, oi, v, odt);
    }
  }
}

// k_down_any for Q6_K down matrices (the 35B's down projections), on the packed-f16 dot instead of a decode to f32.
// Grid (ceil(H / 8), T), 512 threads, one output row a wavefront: eight rows share one staging of the token's h (a
// four-row workgroup read more h than weights at decode width, 12.6 MB against 10.3 at k 8, I 768, H 2048). The
// token's k x I / 32 (expert, chunk) items go up to four a lane, every weight load issued before h is staged, so the
// weights' round trip overlaps the staging. h comes in one of two forms:
//   PREP = false: fp32 [T k][I], staged as f16 pairs in natural order (weights 2m, 2m + 1);
//   PREP = true: prepared rows [T k][I / 64 * 36] in the Q4_K order (lmoe_moe_gate_up with a Q6_K down: dword
//     4 i + s of a 64-value unit holds values (4 i, 4 i + 2) + 32 (s & 1) for s < 2, (4 i + 1, 4 i + 3) + 32 (s & 1)
//     for s >= 2), copied as they are with 16-byte loads: 2.25 bytes a value against 4.
// A chunk's 6-bit q (ql nibble | qh bits << 4) go four to a dword; v_perm spreads two of them to the low byte of each
// half and one shift-or makes the f16 pair (64 + q_a, 64 + q_b), from which one packed subtraction of 96 leaves
// q - 32 exact; v_dot2 then forms sum h (q - 32) over each 16-weight scale group, times (d sc). About 13 VALU for 4
// weights against ~30 for the f32 decode; results are within rounding of k_down_any's (h rounded to f16 once, as
// the Q4 down kernels take it). Items past 256 a row take further passes.
constexpr int kQ6Slots = 4;
template <bool PREP>
__global__ void __launch_bounds__(512)
    k_down_q6k(const void *hin, const uint32_t *ids, const float *scores, int k, const uint8_t *wd, int n_experts,
               int I, int H, size_t rbd, const float *shared, const float *gate, int gate_stride,
               const void *residual, int rdt, void *out, int odt) {
  extern __shared__ uint32_t hl[];  // the token's h: k rows of I / 2 dwords (natural) or I / 64 * 36 (prepared)
  __shared__ uint32_t eid[32];
  __shared__ float esc[32];
  const int t = blockIdx.y;
  const int rowd = PREP ? I / 64 * 36 : I / 2;  // dwords a staged h row
  if (threadIdx.x < k) {
    eid[threadIdx.x] = ids[size_t(t) * k + threadIdx.x];
    esc[threadIdx.x] = scores ? scores[size_t(t) * k + threadIdx.x] : 1.0f;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int o0 = blockIdx.x * 8 + wave;  // this wavefront's output row (past H: row H - 1 again, not stored)
  const int o = min(o0, H - 1);
  const int nch = I / 32, n = k * nch;
  uint32_t lq[kQ6Slots][8], hq[kQ6Slots][8], scw[kQ6Slots];
  float dd[kQ6Slots], sc[kQ6Slots];
  int jj[kQ6Slots], cc[kQ6Slots];
  // slots a pass: only as many as a lane of the wavefront has items for (uniform), so that short rows (the
  // decode chain's one slot a row: 24 items at I 768) do not decode whole wavefronts of repeats
  int ns = kQ6Slots;
  // item u = j (I / 32) + c: chunk c of expert j; slot q holds u0 + 64 q (clamped repeats weigh 0)
  auto load = [&](int u0) {
    ns = min(kQ6Slots, (n - (u0 - lane) + 63) / 64);
#pragma unroll
    for (int q = 0; q < kQ6Slots; ++q) {
      if (q >= ns) break;
      const int u = min(u0 + 64 * q, n - 1), j = u / nch, c = u - j * nch;
      const uint32_t e = eid[j];
      sc[q] = u0 + 64 * q < n && e < uint32_t(n_experts) ? esc[j] : 0.0f;
      jj[q] = j;
      cc[q] = c;
      const int js = c & 7, hh = js >> 2, g = js & 3;
      const uint8_t *b = wd + (size_t(e < uint32_t(n_experts) ? e : 0u) * H + o) * rbd + size_t(c >> 3) * 210;
      load_window8(b + 64 * hh + 32 * (g & 1), lq[q]);
      load_window8(b + 128 + 32 * hh, hq[q]);
      dd[q] = f16at(b + 208);
      scw[q] = ld16(b + 192 + 8 * hh + 2 * g);
    }
  };
  float acc = 0.0f;
  const h2_t k96 = {_Float16(96.0f), _Float16(96.0f)};
  auto compute = [&]() {
#pragma unroll
    for (int q = 0; q < kQ6Slots; ++q) {
      if (q >= ns) break;
      const int c = cc[q], g = (c & 7) & 3, sl = 4 * (g >> 1), shh = 2 * g;
      // the chunk's h pairs: natural, 16 dwords from 16 c; prepared, unit c / 2's dwords, half c & 1
      const uint32_t *hp = hl + jj[q] * rowd + (PREP ? 36 * (c >> 1) + (c & 1) : 16 * c);
      float g0 = 0.0f, g1 = 0.0f;  // sum h (q - 32) over the chunk's two scale groups (weights 0-15, 16-31)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t q6 = ((lq[q][i] >> sl) & 0x0F0F0F0Fu) | (((hq[q][i] >> shh) & 0x03030303u) << 4);
        // weights 4 i .. 4 i + 3: natural pairs (0, 1), (2, 3); prepared pairs (0, 2), (1, 3)
        const uint32_t pa = (__builtin_amdgcn_perm(0u, q6, PREP ? 0x0C020C00u : 0x0C010C00u) << 4) | 0x54005400u;
        const uint32_t pb = (__builtin_amdgcn_perm(0u, q6, PREP ? 0x0C030C01u : 0x0C030C02u) << 4) | 0x54005400u;
        const uint32_t wa = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, pa) - k96);
        const uint32_t wb = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, pb) - k96);
        float &gi = i < 4 ? g0 : g1;
        gi = dot2(wa, PREP ? hp[4 * i] : hp[2 * i], gi);
        gi = dot2(wb, PREP ? hp[4 * i + 2] : hp[2 * i + 1], gi);
      }
      const float d = dd[q];
      const float ds0 = d * float(int(int8_t(uint8_t(scw[q])))), ds1 = d * float(int(int8_t(uint8_t(scw[q] >> 8))));
      acc = fmaf(sc[q], ds0 * g0 + ds1 * g1, acc);
    }
  };
  load(lane);  // the first four items' weights go out before h is staged
  if (PREP) {  // k prepared rows, contiguous, copied as they are
    const u32x4 *src = reinterpret_cast<const u32x4 *>(static_cast<const uint32_t *>(hin) + size_t(t) * k * rowd);
    u32x4 *dst = reinterpret_cast<u32x4 *>(hl);
    for (int i = threadIdx.x; i < k * rowd / 4; i += 512) dst[i] = src[i];
  } else {
    const float2 *src = reinterpret_cast<const float2 *>(static_cast<const float *>(hin) + size_t(t) * k * I);
    for (int i = threadIdx.x; i < k * I / 2; i += 512) {
      const float2 v = src[i];
      const h2_t p = {_Float16(v.x), _Float16(v.y)};
      hl[i] = __builtin_bit_cast(uint32_t, p);
    }
  }
  __syncthreads();
  compute();
  for (int u0 = lane + 64 * kQ6Slots; u0 - lane < n; u0 += 64 * kQ6Slots) {
    load(u0);
    compute();
  }
  float v = wave_sum(acc);
  if (lane == 0 && o0 < H) {
    const size_t oi = size_t(t) * H + o0;
    if (shared) v += sigmoidf_(gate[size_t(t) * gate_stride]) * shared[oi];
    if (residual) v += load_elt(residual, oi, rdt);
    store_elt(out, oi, v, odt);
  }
}

// The Q8_0 down on h prepared in the Q4_0 order (lmoe_moe_gate_up with a Q8_0 down; values (4 i, 4 i + 2) + 16 (s & 1)
// of a 32-value span in dword 4 i + s for s < 2, (4 i + 1, 4 i + 3) + 16 (s & 1) for s >= 2), in k_down_q6k's shape:
// one output row a wavefront, 8 a workgroup, up to four (expert, block) items a lane with every weight load out
// before h is staged. A block's 34 bytes are 2-byte aligned: 9 dwords from the 4-byte aligned address at or below
// it (with K a multiple of 64 a row holds an even number of blocks, so a row's last block starts 2 mod 4 and the
// window ends inside the row). Each int8 q becomes the exact f16 1024 + (q + 128) through one xor and the 0x64
// byte of v_perm, one packed subtraction of 1152 leaves q, and v_dot2 forms sum h q over the block, times d.
constexpr int kQ8Slots = 4;
__global__ void __launch_bounds__(512)
    k_down_q8p(const uint32_t *hprep, const uint32_t *ids, const float *scores, int k, const uint8_t *wd,
               int n_experts, int I, int H, size_t rbd, const float *shared, const float *gate, int gate_stride,
               const void *residual, int rdt, void *out, int odt) {
  extern __shared__ uint32_t hl[];  // the token's k prepared h rows, I / 64 * 36 dwords each
  __shared__ uint32_t eid[32];
  __shared__ float esc[32];
  const int t = blockIdx.y;
  const int rowd = I / 64 * 36;
  if (threadIdx.x < k) {
    eid[threadIdx.x] = ids[size_t(t) * k + threadIdx.x];
    esc[threadIdx.x] = scores ? scores[size_t(t) * k + threadIdx.x] : 1.0f;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int o0 = blockIdx.x * 8 + wave;  // this wavefront's output row (past H: row H - 1 again, not stored)
  const int o = min(o0, H - 1);
  const int nch = I / 32, n = k * nch;
  uint32_t qw[kQ8Slots][8];
  float dd[kQ8Slots], sc[kQ8Slots];
  int jj[kQ8Slots], cc[kQ8Slots];
  int ns = kQ8Slots;
  auto load = [&](int u0) {
    ns = min(kQ8Slots, (n - (u0 - lane) + 63) / 64);
#pragma unroll
    for (int q = 0; q < kQ8Slots; ++q) {
      if (q >= ns) break;
      const int u = min(u0 + 64 * q, n - 1), j = u / nch, c = u - j * nch;
      const uint32_t e = eid[j];
      sc[q] = u0 + 64 * q < n && e < uint32_t(n_experts) ? esc[j] : 0.0f;
      jj[q] = j;
      cc[q] = c;
      const uintptr_t a = reinterpret_cast<uintptr_t>(
          wd + (size_t(e < uint32_t(n_experts) ? e : 0u) * H + o) * rbd + size_t(c) * 34);
      const uint32_t *base = reinterpret_cast<const uint32_t *>(a & ~uintptr_t(3));
      const u32x4a4 v0 = *reinterpret_cast<const u32x4a4 *>(base), v1 = *reinterpret_cast<const u32x4a4 *>(base + 4);
      const uint32_t w[9] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w, base[8]};
      const bool odd = (a & 2) != 0;  // the block starts 2 mod 4: d in the high half of w[0], qs from w[1]
      dd[q] = float(__builtin_bit_cast(_Float16, uint16_t(odd ? w[0] >> 16 : w[0] & 0xFFFFu)));
#pragma unroll
      for (int i = 0; i < 8; ++i) qw[q][i] = odd ? w[i + 1] : __builtin_amdgcn_alignbyte(w[i + 1], w[i], 2);
    }
  };
  float acc = 0.0f;
  const h2_t k1152 = {_Float16(1152.0f), _Float16(1152.0f)};
  auto pair = [&](uint32_t x, uint32_t sel) {  // two bytes of x ^ 0x80.. as f16 1024 + u, less 1152: the int8 q
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(0x64646464u, x, sel)) - k1152);
  };
  auto compute = [&]() {
#pragma unroll
    for (int q = 0; q < kQ8Slots; ++q) {
      if (q >= ns) break;
      const int c = cc[q];
      const uint32_t *hp = hl + jj[q] * rowd + 36 * (c >> 1) + 16 * (c & 1);
      float sm = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {  // weights 4 i .. 4 i + 3 (word i) and 16 + 4 i .. (word 4 + i)
        const uint32_t lo = qw[q][i] ^ 0x80808080u, hi = qw[q][4 + i] ^ 0x80808080u;
        sm = dot2(pair(lo, 0x04020400u), hp[4 * i], sm);
        sm = dot2(pair(hi, 0x04020400u), hp[4 * i + 1], sm);
        sm = dot2(pair(lo, 0x04030401u), hp[4 * i + 2], sm);
        sm = dot2(pair(hi, 0x04030401u), hp[4 * i + 3], sm);
      }
      acc = fmaf(sc[q], dd[q] * sm, acc);
    }
  };
  load(lane);  // the first four items' weights go out before h is staged
  {
    const u32x4 *src = reinterpret_cast<const u32x4 *>(hprep + size_t(t) * k * rowd);
    u32x4 *dst = reinterpret_cast<u32x4 *>(hl);
    for (int i = threadIdx.x; i < k * rowd / 4; i += 512) dst[i] = src[i];
  }
  __syncthreads();
  compute();
  for (int u0 = lane + 64 * kQ8Slots; u0 - lane < n; u0 += 64 * kQ8Slots) {
    load(u0);
    compute();
  }
  float v = wave_sum(acc);
  if (lane == 0 && o0 < H) {
    const size_t oi = size_t(t) * H + o0;
    if (shared) v += sigmoidf_(gate[size_t(t) * gate_stride]) * shared[oi];
    if (residual) v += load_elt(residual, oi, rdt);
    store_elt(out, oi, v, odt);
  }
}

// One thread a 32-weight chunk: q[c][r][32 u .. 32 u + 31] of the expert at slots[c] (identity when slots is
// null), in natural order or, with kperm, in the grouped GEMMs' K order (4-element groups 0-3, 16-19, 4-7, 20-23,
// 8-11, 24-27, 12-15, 28-31 of every 32). Slots past the experts give zeros.
template <int T>
__global__ void __launch_bounds__(256) k_dequant_any(const uint8_t *buf, int n_experts, int rows, int cols,
                                                     size_t rb, const uint32_t *slots, int n, void *q, int odt,
                                                     int kperm) {
  const int U = cols / 32;
  const size_t gid = size_t(blockIdx.x) * 256 + threadIdx.x;
  if (gid >= size_t(n) * rows * U) return;
  const int u = int(gid % U);
  const size_t rc = gid / U;
  const int r = int(rc % rows), c = int(rc / rows);
  const uint32_t e = slots ? slots[c] : uint32_t(c);
  const size_t o = (size_t(c) * rows + r) * cols + 32 * size_t(u);
  float w[32];
  if (e < uint32_t(n_experts)) {
    decode32<T>(buf + (size_t(e) * rows + r) * rb, u, w);
  } else {
#pragma unroll
    for (int i = 0; i < 32; ++i) w[i] = 0.0f;
  }
  if (odt == LMOE_F16) {
    // four 16-byte stores: K-order block p holds natural groups p and p + 4 (elements 4p.., 16 + 4p..), natural
    // block p elements 8p .. 8p + 7
    u32x4 *dst = reinterpret_cast<u32x4 *>(static_cast<_Float16 *>(q) + o);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int a = kperm ? 4 * p : 8 * p, b = kperm ? 16 + 4 * p : 8 * p + 4;
      uint32_t v[4];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        v[i] = __builtin_bit_cast(uint32_t, h2_t{_Float16(w[a + 2 * i]), _Float16(w[a + 2 * i + 1])});
        v[2 + i] = __builtin_bit_cast(uint32_t, h2_t{_Float16(w[b + 2 * i]), _Float16(w[b + 2 * i + 1])});
      }
      dst[p] = u32x4{v[0], v[1], v[2], v[3]};
    }
    return;
  }
#pragma unroll
  for (int g4 = 0; g4 < 8; ++g4) {
    const int at = kperm ? (g4 < 4 ? 8 * g4 : 8 * (g4 - 4) + 4) : 4 * g4;
#pragma unroll
    for (int i = 0; i < 4; ++i) store_elt(q, o + at + i, w[4 * g4 + i], odt);
  }
}

static int check_any(const char *fn, int type, int rows, int cols, const void *buf) {
  LMOE_REQUIRE(qtype_any(type), LMOE_ETYPE,
               "%s: ggml type %d is not supported (Q4_0 = 2, Q4_1 = 3, Q8_0 = 8, Q4_K = 12, Q5_K = 13, Q6_K = 14)",
               fn, type);
  LMOE_REQUIRE(rows > 0 && cols > 0 && cols % block_weights_any(type) == 0, LMOE_ESHAPE,
               "%s: row length %d is not a multiple of %d", fn, cols, block_weights_any(type));
  LMOE_REQUIRE(buf && (reinterpret_cast<uintptr_t>(buf) % block_align(type)) == 0, LMOE_EALIGN,
               "%s: ggml type %d buffers must be %d-byte aligned", fn, type, block_align(type));
  return 0;
}

static size_t row_bytes_any(int type, int cols) {
  return size_t(cols / block_weights_any(type)) * block_bytes_any(type);
}

int gate_up_any(const char *fn, const void *x, int xdt, const uint32_t *slots, int n_slots, int topk,
                const uint8_t *wg, const uint8_t *wu, int tg, int tu, int n_experts, int H, int I, float *h,
                hipStream_t st) {
  if (int rc = check_any(fn, tg, I, H, wg)) return rc;
  if (int rc = check_any(fn, tu, I, H, wu)) return rc;
  LMOE_REQUIRE(H % 32 == 0 && size_t(H) * 4 <= 160 * 1024, LMOE_ESHAPE,
               "%s: hidden size %d is above the 40960 this kernel stages", fn, H);
  LMOE_REQUIRE(I % 2 == 0, LMOE_ESHAPE, "%s: %d rows is not even", fn, I);
  if (n_slots == 0) return 0;
  LMOE_REQUIRE(n_slots <= 65535, LMOE_ESHAPE, "%s: %d slots a call is above the 65535 this kernel takes", fn,
               n_slots);
  LMOE_REQUIRE(x && slots && h, LMOE_EINVAL, "%s: null pointer", fn);
  const size_t lds = size_t(H) * 4;
  if (int rc = allow_lds(k_gate_up_any, lds, fn)) return rc;
  launch(k_gate_up_any, dim3((I + 4 * kAnyRows - 1) / (4 * kAnyRows), n_slots), dim3(256), lds, st, x, xdt, slots,
         topk, wg, wu, tg, tu, n_experts, H, I, row_bytes_any(tg, H), row_bytes_any(tu, H), h);
  LMOE_LAUNCHED(fn);
  return 0;
}

int down_any(const char *fn, const float *h, const uint32_t *ids, const float *scores, int T, int k,
             const uint8_t *wd, int td, int n_experts, int I, int H, const float *shared, const float *gate,
             int gate_stride, const void *residual, int rdt, void *out, int odt, hipStream_t st) {
  if (int rc = check_any(fn, td, H, I, wd)) return rc;
  LMOE_REQUIRE(H % 2 == 0, LMOE_ESHAPE, "%s: %d rows is not even", fn, H);
  const size_t lds = size_t(k) * I * 4;
  LMOE_REQUIRE(lds <= 150 * 1024, LMOE_ESHAPE, "%s: k %d rows of width %d exceed the LDS this kernel stages", fn, k,
               I);
  if (T == 0) return 0;
  LMOE_REQUIRE(T <= 65535, LMOE_ESHAPE, "%s: %d tokens a call is above the 65535 this kernel takes", fn, T);
  LMOE_REQUIRE(h && ids && out, LMOE_EINVAL, "%s: null pointer", fn);
  const dim3 grid((H + 4 * kAnyRows - 1) / (4 * kAnyRows), T);
  // a row of more than 64 (expert, chunk) items (the decode layer's k slots a token) takes the flattened forms; the
  // decode chain's one slot a row keeps the serial one
  const bool flat = k * (I / 32) > 64;
  if (flat && td == LMOE_Q6_K) {  // h as f16 pairs: k I 2 bytes
    const size_t lq6 = size_t(k) * I / 2 * 4;
    if (int rc = allow_lds(k_down_q6k<false>, lq6, fn)) return rc;
    launch(k_down_q6k<false>, dim3((H + 7) / 8, T), dim3(512), lq6, st, static_cast<const void *>(h), ids, scores, k,
           wd, n_experts, I, H, row_bytes_any(td, I), shared, gate, gate_stride, residual, rdt, out, odt);
    LMOE_LAUNCHED(fn);
    return 0;
  }
  auto kern = flat ? k_down_any<true> : k_down_any<false>;
  if (int rc = allow_lds(kern, lds, fn)) return rc;
  launch(kern, grid, dim3(256), lds, st, h, ids, scores, k, wd, td, n_experts, I, H, row_bytes_any(td, I), shared,
         gate, gate_stride, residual, rdt, out, odt);
  LMOE_LAUNCHED(fn);
  return 0;
}

// The Q6_K / Q8_0 down + combine on prepared h rows [T k][I / 64 * 36] in the Q4_K / Q4_0 order
// (lmoe_gemv_down_combine_prepped with such a down matrix; the rows' sum dwords are not read).
int down_packed_prepped(const char *fn, int td, const uint32_t *hprep, const uint32_t *ids, const float *scores,
                        int T, int k, const uint8_t *wd, int n_experts, int I, int H, const float *shared,
                        const float *gate, int gate_stride, const void *residual, int rdt, void *out, int odt,
                        hipStream_t st) {
  LMOE_REQUIRE(td == LMOE_Q6_K || td == LMOE_Q8_0, LMOE_ETYPE, "%s: prepared h takes a Q4_0 / Q4_K / Q6_K / Q8_0 "
               "down (got ggml type %d)", fn, td);
  if (int rc = check_any(fn, td, H, I, wd)) return rc;
  LMOE_REQUIRE(I % 64 == 0, LMOE_ESHAPE, "%s: width %d is not a multiple of 64", fn, I);
  LMOE_REQUIRE(td != LMOE_Q8_0 || (reinterpret_cast<uintptr_t>(wd) & 3) == 0, LMOE_EALIGN,
               "%s: Q8_0 experts must be 4-byte aligned here", fn);
  LMOE_REQUIRE(dtype_ok(odt) && (!residual || dtype_ok(rdt)), LMOE_EINVAL, "%s: bad dtype", fn);
  LMOE_REQUIRE(k > 0 && k <= 32 && n_experts > 0, LMOE_ESHAPE, "%s: k %d of %d experts", fn, k, n_experts);
  LMOE_REQUIRE(!shared == !gate, LMOE_EINVAL, "%s: shared and gate go together", fn);
  const size_t lds = size_t(k) * (I / 64) * 36 * 4;
  LMOE_REQUIRE(lds <= 150 * 1024, LMOE_ESHAPE, "%s: k %d rows of width %d exceed the LDS this kernel stages", fn, k,
               I);
  if (T == 0) return 0;
  LMOE_REQUIRE(T <= 65535, LMOE_ESHAPE, "%s: %d tokens a call is above the 65535 this kernel takes", fn, T);
  LMOE_REQUIRE(hprep && ids && out, LMOE_EINVAL, "%s: null pointer", fn);
  LMOE_REQUIRE(aligned16(hprep), LMOE_EALIGN, "%s: prepared h must be 16-byte aligned", fn);
  if (td == LMOE_Q8_0) {
    if (int rc = allow_lds(k_down_q8p, lds, fn)) return rc;
    launch(k_down_q8p, dim3((H + 7) / 8, T), dim3(512), lds, st, hprep, ids, scores, k, wd, n_experts, I, H,
           row_bytes_any(td, I), shared, gate, gate_stride, residual, rdt, out, odt);
    LMOE_LAUNCHED(fn);
    return 0;
  }
  if (int rc = allow_lds(k_down_q6k<true>, lds, fn)) return rc;
  launch(k_down_q6k<true>, dim3((H + 7) / 8, T), dim3(512), lds, st, static_cast<const void *>(hprep), ids, scores,
         k, wd, n_experts, I, H, row_bytes_any(LMOE_Q6_K, I), shared, gate, gate_stride, residual, rdt, out, odt);
  LMOE_LAUNCHED(fn);
  return 0;
}

int dequant_any(const char *fn, const uint8_t *buf, int type, int n_experts, int rows, int cols,
                const uint32_t *slots, int n, void *q, int odt, int kperm, hipStream_t st) {
  if (int rc = check_any(fn, type, rows, cols, buf)) return rc;
  LMOE_REQUIRE(dtype_ok(odt), LMOE_EINVAL, "%s: bad dtype", fn);
  LMOE_REQUIRE(n >= 0 && n_experts > 0, LMOE_ESHAPE, "%s: bad shape", fn);
  if (n == 0) return 0;
  LMOE_REQUIRE(q, LMOE_EINVAL, "%s: null pointer", fn);
  const size_t chunks = size_t(n) * rows * (cols / 32);
  const dim3 grid(unsigned((chunks + 255) / 256));
  const size_t rb = row_bytes_any(type, cols);
  auto go = [&](auto kern) { launch(kern, grid, dim3(256), 0, st, buf, n_experts, rows, cols, rb, slots, n, q, odt, kperm); };
  switch (type) {
    case LMOE_Q4_0: go(k_dequant_any<LMOE_Q4_0>); break;
    case LMOE_Q4_1: go(k_dequant_any<LMOE_Q4_1>); break;
    case LMOE_Q8_0: go(k_dequant_any<LMOE_Q8_0>); break;
    case LMOE_Q4_K: go(k_dequant_any<LMOE_Q4_K>); break;
    case LMOE_Q5_K: go(k_dequant_any<LMOE_Q5_K>); break;
    default: go(k_dequant_any<LMOE_Q6_K>); break;
  }
  LMOE_LAUNCHED(fn);
  return 0;
}

}  // namespace lmoe

using namespace lmoe;

extern "C" int lmoe_dequant_gemm_f16(const uint8_t *buf, int type, int n_experts, int rows, int cols, void *out,
                                     void *stream) {
  return dequant_any("lmoe_dequant_gemm_f16", buf, type, n_experts, rows, cols, nullptr, n_experts, out, LMOE_F16, 1,
                     (hipStream_t)stream);
}
