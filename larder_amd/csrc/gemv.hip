// Decode chain: gate/up + SwiGLU, and down + weighted combine, reading GGUF Q4_0 / Q4_K blocks in place.
//
// The reference runs these as gguf_gate_up / gguf_down (gguf_experts.py:452-526): LPR lanes a row, 16-bit loads
// of each 18-byte block, shuffle-tree reductions. Here, for CDNA4:
//   * each wavefront takes a task of 4 consecutive rows of one expert matrix (gate and up together), which is one
//     contiguous byte range of 144 * P bytes (P = row length / 64). Its 16-byte loads are issued first, into
//     registers, so the HBM round trip overlaps the staging of the activations; they land in the wavefront's own
//     LDS region and are read back as 36-byte "units" (64 weights: two Q4_0 blocks or a quarter Q4_K
//     super-block), each lane a unit, 9 dword reads at a 9-dword lane stride (bank-conflict free);
//   * activations arrive prepared (f16 pairs in nibble order plus half-unit sums, lmoe_common.h) and are copied
//     into LDS as they are; gate/up writes h prepared for down the same way. Raw activations are also accepted
//     and rearranged in LDS by the workgroup;
//   * each unit's nibbles meet the activations in v_dot2_f32_f16, fp32 accumulation; per-unit partial sums go to
//     LDS and are added in a fixed order, the last steps on DPP (deterministic results);
//   * down adds the k experts of a token, weighted by the router scores, plus the shared expert and a residual,
//     in the same kernel, so no [T * k, H] intermediate is written.
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "lmoe_common.h"

namespace lmoe {


__device__ __forceinline__ int elt_size(int dt) { return dt == LMOE_F32 ? 4 : 2; }

// ndw dwords (a multiple of 4, 16-byte aligned) from global src to LDS dst, 16 bytes a thread a step. A thread's
// loads go out 8 at a time, none predicated (indices clamped to the last chunk), ahead of its stores, so their
// round trips overlap instead of queueing one behind the other.
__device__ __forceinline__ void copy_to_lds(const void *src, void *dst, int ndw, int tid, int nthr) {
  const u32x4 *s = static_cast<const u32x4 *>(src);
  u32x4 *d = static_cast<u32x4 *>(dst);
  const int n = ndw / 4;
  for (int b = tid; b < n; b += 8 * nthr) {
    u32x4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = s[min(b + j * nthr, n - 1)];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (b + j * nthr < n) d[b + j * nthr] = v[j];
  }
}

__device__ __forceinline__ float lds_elt(const void *raw, int i, int dt) {
  if (dt == LMOE_F32) return static_cast<const float *>(raw)[i];
  const uint16_t b = static_cast<const uint16_t *>(raw)[i];
  return dt == LMOE_F16 ? float(__builtin_bit_cast(_Float16, b)) : bf16_to_f32(b);
}

// A raw activation row in LDS (64 P values of dtype dt) -> prepared units (pairs and sums) in LDS.
template <int TQ>
__device__ __forceinline__ void prep_in_lds(const void *raw, int dt, int P, uint32_t *xs, int tid, int nthr) {
  for (int idx = tid; idx < XS * P; idx += nthr) {
    const int p = idx / XS, dw = idx - p * XS;
    xs[idx] = prep_dword<TQ>([&](int i) { return lds_elt(raw, i, dt); }, p, dw);
  }
}

// The half-unit sums of prepared units written without them, from their pairs: a unit's first 32 weights sit in
// dwords 0..15 (Q4_0) or in the even dwords (Q4_K).
template <int TQ>
__device__ __forceinline__ void sums_in_lds(uint32_t *xs, int units, int tid, int nthr) {
  for (int hu = tid; hu < 2 * units; hu += nthr) {
    const int p = hu >> 1, half = hu & 1;
    const uint32_t *u = xs + p * XS;
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t w = TQ == LMOE_Q4_K ? u[2 * i + half] : u[16 * half + i];
      s += half_lo(w) + half_hi(w);
    }
    xs[p * XS + 32 + half] = __builtin_bit_cast(uint32_t, s);
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

// The dot of unit p of a staged row (9 P dwords) with a prepared unit xu (pairs at 0..31, sums at 32, 33).
template <int TQ>
__device__ __forceinline__ float row_unit_dot(const uint32_t *row, int p, const uint32_t *xu) {
  uint32_t xv[32];
  load_x32(xu, xv);
  const float sx0 = __builtin_bit_cast(float, xu[32]), sx1 = __builtin_bit_cast(float, xu[33]);
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
// Activations: prepared rows xg (and xu, for an up type other than gate's), or raw rows x of dtype xdt when xg is
// null. Outputs: h (fp32, [n_slots][I]) and / or hprep (prepared rows of width I for block type td, pairs only:
// the consumer derives the sums).
// LDS: the prepared unit rows (gate's, then up's when the types differ), then a region that first holds the raw x
// row (raw input only) and then each wavefront's 8 staged weight rows, then each wavefront's 8 x (P + 1) partials.
template <int TG, int TU, int RB, int NC, int NW>
__global__ void __launch_bounds__(64 * NW, 3)
    k_gate_up(const uint32_t *xg_prep, const uint32_t *xu_prep, const void *x, int xdt, const uint32_t *slots,
              int topk, const uint8_t *wg, const uint8_t *wu, int n_experts, int I, float *h, uint32_t *hprep,
              int td, int P, const float *logits, int ld_stride, int norm, uint32_t *ids_out, float *scores_out) {
  constexpr bool SAME = TG == TU;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int s = blockIdx.y;
  const int r0 = (blockIdx.x * NW + wave) * RB;
  uint32_t e;
  if (logits) {  // the router's top-k of this slot's token, by wavefront 0, the slot's pick through LDS
    __shared__ uint32_t pick_id[32];
    __shared__ float pick_sc[32];
    __shared__ __attribute__((aligned(16))) uint32_t scr[64];
    if (wave == 0) {
      const float *row = logits + size_t(s / topk) * ld_stride;
      auto run = [&](auto npl) {
        constexpr int N = decltype(npl)::value;
        float v[N];
#pragma unroll
        for (int j = 0; j < N; ++j) v[j] = lane + 64 * j < n_experts ? row[lane + 64 * j] : -INFINITY;
        uint32_t id;
        float sc;
        topk_wave<N>(v, n_experts, topk, norm, scr, &id, &sc);
        if (lane < topk) {
          pick_id[lane] = id;
          pick_sc[lane] = sc;
        }
      };
      if (n_experts <= 64)
        run(std::integral_constant<int, 1>());
      else if (n_experts <= 128)
        run(std::integral_constant<int, 2>());
      else if (n_experts <= 256)
        run(std::integral_constant<int, 4>());
      else if (n_experts <= 512)
        run(std::integral_constant<int, 8>());
      else
        run(std::integral_constant<int, 16>());
    }
    __syncthreads();
    e = pick_id[s % topk];
    if (blockIdx.x == 0 && threadIdx.x == 0) {
      ids_out[s] = e;
      scores_out[s] = pick_sc[s % topk];
    }
  } else {
    e = slots[s];
  }
  extern __shared__ u32x4 lds4[];
  uint32_t *xg = reinterpret_cast<uint32_t *>(lds4);
  uint32_t *xu = SAME ? xg : xg + P * XS;
  uint32_t *region = xu + P * XS;
  const int stage_dw = 2 * RB * 9 * P;
  const int xraw_dw = xg_prep ? 0 : 16 * P * elt_size(xdt);  // 64 P elements
  uint32_t *stage = region + wave * stage_dw;
  float *red = reinterpret_cast<float *>(region + max(NW * stage_dw, xraw_dw)) + wave * (2 * RB * (P + 1));
  const bool valid = e < uint32_t(n_experts);  // no such expert: zero rows (cpu_kern.cpp:316-318)

  // 1) this wavefront's 2 RB rows, RB 9 P / 4 16-byte chunks a matrix, into registers. The loads are not
  // predicated (a lane past the end re-reads the last chunk; a wavefront with no rows or no expert reads expert 0's
  // last row block), so they issue back to back with no wait between them.
  const int C = RB * 9 * P / 4;
  const size_t rowb = size_t(36) * P;
  const size_t rsafe = size_t(valid ? e : 0u) * I + min(r0, I - RB);
  const u32x4 *gsrc = reinterpret_cast<const u32x4 *>(wg + rsafe * rowb);
  const u32x4 *usrc = reinterpret_cast<const u32x4 *>(wu + rsafe * rowb);
  u32x4 vg[NC], vu[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = min(lane + 64 * i, C - 1);
    vg[i] = __builtin_nontemporal_load(gsrc + c);
    vu[i] = __builtin_nontemporal_load(usrc + c);
  }
  // 2) the activation row
  const size_t xrow = size_t(s / topk);
  if (xg_prep) {
    copy_to_lds(xg_prep + xrow * P * XS, xg, P * XS, threadIdx.x, 64 * NW);
    if (!SAME) copy_to_lds(xu_prep + xrow * P * XS, xu, P * XS, threadIdx.x, 64 * NW);
    __syncthreads();
  } else {
    copy_to_lds(static_cast<const char *>(x) + xrow * 64 * P * elt_size(xdt), region, 16 * P * elt_size(xdt),
                threadIdx.x, 64 * NW);
    __syncthreads();
    prep_in_lds<TG>(region, xdt, P, xg, threadIdx.x, 64 * NW);
    if (!SAME) prep_in_lds<TU>(region, xdt, P, xu, threadIdx.x, 64 * NW);
    __syncthreads();
  }
  if (r0 >= I) return;
  if (!valid) {
    if (lane < RB) {
      if (h) h[size_t(s) * I + r0 + lane] = 0.0f;
      if (hprep) {
        int dw, half;
        const int n = r0 + lane;
        xslot(n & 63, td == LMOE_Q4_K ? 32 : 16, &dw, &half);
        reinterpret_cast<_Float16 *>(hprep + (size_t(s) * (I / 64) + (n >> 6)) * XS + dw)[half] = _Float16(0.0f);
      }
    }
    return;
  }
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
#pragma unroll 2
  for (int u = lane; u < U; u += 64) {
    const int row = u / P, p = u - row * P;
    float part;
    if (row < RB)
      part = row_unit_dot<TG>(stage + row * 9 * P, p, xg + p * XS);
    else
      part = row_unit_dot<TU>(stage + row * 9 * P, p, xu + p * XS);
    red[row * (P + 1) + p] = part;
  }
  __builtin_amdgcn_wave_barrier();

  // 2 RB rows x P partials: LPR lanes a row, fixed order
  constexpr int LPR = 64 / (2 * RB);
  const int rr = lane / LPR, sub = lane % LPR;
  float acc = 0.0f;
  for (int p = sub; p < P; p += LPR) acc += red[rr * (P + 1) + p];
  acc = LPR == 8 ? sum8(acc) : sum16(acc);
  const float up = lane_xor32(acc);  // up row rr sits RB * LPR = 32 lanes above gate row rr
  if (rr < RB && sub == 0) {
    const int n = r0 + rr;
    const float v = silu_mul(acc, up);
    if (h) h[size_t(s) * I + n] = v;
    if (hprep) {
      int dw, half;
      xslot(n & 63, td == LMOE_Q4_K ? 32 : 16, &dw, &half);
      reinterpret_cast<_Float16 *>(hprep + (size_t(s) * (I / 64) + (n >> 6)) * XS + dw)[half] = _Float16(v);
    }
  }
}


// ---- gate/up with the activation unit in registers (H = 64 P, P = 32 or 64; one block type for gate and up) ----
//
// Grid (ceil(I / (4 RB)), n_slots): four wavefronts a workgroup; wavefront w of block (bx, s) takes gate and up
// rows [(4 bx + w) RB, +RB) of expert e(s). The token's prepared activation row comes into LDS once a workgroup
// (one workgroup barrier); lane l then holds unit p = l % P of it in registers (36 dwords) for the rows
// g, g + G, ... of both matrices (g = l / P, G = 64 / P lane groups). The wavefront's weight rows come in with 16-byte
// loads, go to its own LDS region and are read back a 36-byte unit a lane; each row's P partials are summed over
// the lane group on DPP and permlane swaps. NPL > 0: each wavefront picks the slot's expert from the logits itself
// (NPL a lane; softmax scores only in the one wavefront that writes ids / scores, wavefront 0 of the slot's first
// workgroup); NPL = 0: expert ids from slots. Memory order: logits,
// activation chunks, then (once the id is known) the weights, none predicated, so each group goes out back to back.
// ks: slots a token, topk or, with a shared expert folded in (NPL > 0 only), topk + m: then slot topk + j of a token
// is slice j of the shared expert (its intermediate features [j I, (j + 1) I), the whole expert when m = 1), stored
// as expert n_experts + j of wg / wu, and ids_out / scores_out rows hold ks entries, the last m
// (n_experts + j, sigmoid(logits[t][n_experts])) for the down kernel to weight them like routed experts: the shared
// expert's down is linear in its intermediate features, so the m weighted slices sum to the gated shared row.
//
// RAW (slots given, NPL = 0): x comes raw (dtype xdt) and each workgroup prepares its row in LDS with prep_dword,
// the bits lmoe_prep_x writes, so the launch before it is saved: the drop-in chain's form.
template <int TQ, int P, int RB, int NPL, bool RANKWG, bool RAW = false, bool TL = false>
__global__ void __launch_bounds__(256)
    k_gate_up_xr(const uint32_t *xprep, const uint32_t *slots, int topk, const uint8_t *wg, const uint8_t *wu,
                 int n_experts, int I, float *h, uint32_t *hprep, int td, const float *logits, int ld_stride,
                 int norm, uint32_t *ids_out, float *scores_out, int ks, const void *x, int xdt,
                 unsigned long long *tl) {
  constexpr int NW = 4, G = 64 / P, RG = RB / G;
  static_assert(P == 32 || P == 64, "32 or 64 units a row");
  static_assert(RB % G == 0, "rows split evenly over the lane groups");
  static_assert(!RAW || NPL == 0, "raw x: slots given");
  static_assert(!RAW || NW * 2 * RB * 9 * P >= 64 * P, "the stages hold the raw row (f32 at most)");
  static_assert(!TL || (!RAW && !RANKWG), "stamps in the per-wavefront pick form only");
  tl_stamp<TL>(tl, 0);
  constexpr int C = RB * 9 * P / 4;  // 16-byte chunks of RB rows of one matrix
  constexpr int NC2 = (2 * C + 63) / 64;  // of both matrices' rows, a lane
  constexpr int STAGE = 2 * RB * 9 * P;  // dwords a wavefront
  constexpr int XC = 9 * P;              // 16-byte chunks of the prepared activation row
  constexpr int NT = 64 * NW;
  constexpr int XPT = (XC + NT - 1) / NT;  // of them a thread
  // LDS (16-byte chunks): the activation row, NW stages, NW x 64 dwords of top-k scratch
  __shared__ u32x4 lds4[XC + NW * (STAGE / 4) + NW * 16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int s = blockIdx.y;
  const int r0 = (blockIdx.x * NW + wave) * RB;
  const int g = lane / P, p = lane % P;
  u32x4 *xl = lds4;
  uint32_t *stage = reinterpret_cast<uint32_t *>(lds4 + XC) + wave * STAGE;
  uint32_t *scr = reinterpret_cast<uint32_t *>(lds4 + XC + NW * (STAGE / 4)) + wave * 64;
  const size_t xrow = size_t(s / ks);
  const int jslot = s % ks;
  const bool shared_slot = NPL > 0 && jslot >= topk;  // uniform across the workgroup

  // RANKWG and E <= 512: the workgroup ranks its token's logits once (rank256: the four wavefronts share the
  // comparisons); otherwise each wavefront ranks them itself (topk_wave)
  constexpr bool RANK = RANKWG && NPL > 0 && NPL <= 8;
  __shared__ __attribute__((aligned(16))) RankScratch rs;
  float v[NPL > 0 ? NPL : 1];
  float lv[2];
  uint32_t e = 0;
  // RAW: the raw x row, over the stages (written only after the row is prepared)
  u32x4 *xraw = lds4 + XC;
  constexpr int XRR = RAW ? (16 * P + NT - 1) / NT : 1;  // raw 16-byte chunks a thread (f32 at most)
  u32x4 xr4[XRR];
  if (RAW) {  // the raw row's chunks first, then the slot's expert
    const int xch = xdt == LMOE_F32 ? 16 * P : 8 * P;
    const u32x4 *xs4 = reinterpret_cast<const u32x4 *>(static_cast<const char *>(x) + xrow * (size_t(xch) * 16));
#pragma unroll
    for (int i = 0; i < XRR; ++i) xr4[i] = xs4[min(int(threadIdx.x) + NT * i, xch - 1)];
    e = slots[s];
  } else if (RANK) {
    const float *row = logits + xrow * ld_stride;
#pragma unroll
    for (int j = 0; j < 2; ++j) lv[j] = row[min(int(threadIdx.x) + 256 * j, n_experts - 1)];
  } else if (NPL > 0) {
    const float *row = logits + xrow * ld_stride;
#pragma unroll
    for (int j = 0; j < NPL; ++j) v[j] = row[min(lane + 64 * j, n_experts - 1)];  // lanes past E: masked by topk_wave
  } else {
    e = slots[s];
  }
  // the logits (or the slot id) go out before the activation row: the count of outstanding loads is in order, so
  // the top-k then waits for the logits alone, not for the row behind them
  asm volatile("" ::: "memory");
  const u32x4 *xg4 = reinterpret_cast<const u32x4 *>(xprep + xrow * P * XS);
  u32x4 xc[RAW ? 1 : XPT];
  if (!RAW) {
#pragma unroll
    for (int i = 0; i < XPT; ++i) xc[i] = xg4[min(int(threadIdx.x) + NT * i, XC - 1)];
  }
  if constexpr (TL) {  // the logits row (slots given: the slot's id) in
    if constexpr (NPL > 0)
      asm volatile("" ::"v"(v[0]), "v"(v[NPL > 0 ? NPL - 1 : 0]));
    else
      asm volatile("" ::"v"(e));
    tl_stamp<TL>(tl, 1);
  }
  if (NPL > 0 && shared_slot) {  // a slice of the folded shared expert: no pick; its id and sigmoid-gated weight
    e = uint32_t(n_experts + jslot - topk);
    if (blockIdx.x == 0 && wave == 0 && lane == 0) {
      ids_out[s] = e;
      scores_out[s] = sigmoidf_(logits[xrow * ld_stride + n_experts]);
    }
  } else if (RANK) {  // uniform across the workgroup (the slot is blockIdx.y)
#pragma unroll
    for (int j = 0; j < 2; ++j)
      if (int(threadIdx.x) + 256 * j < n_experts) rs.vals[threadIdx.x + 256 * j] = lv[j];
    __syncthreads();
    const float p = rank256(rs, n_experts, topk, norm, int(threadIdx.x));
    e = rs.pick[jslot];
    if (blockIdx.x == 0 && int(threadIdx.x) == jslot) {
      ids_out[s] = e;
      scores_out[s] = p;
    }
  } else if (NPL > 0) {  // each wavefront picks the slot's expert itself (no barrier before its weight loads)
    constexpr int N = NPL > 0 ? NPL : 1;
    const int j = jslot;
    uint32_t id;
    if (blockIdx.x == 0 && wave == 0) {  // the slot's scores: one wavefront computes and writes them
      float sc;
      topk_wave<N, true>(v, n_experts, topk, norm, scr, &id, &sc);
      if (lane == j) {
        ids_out[s] = id;
        scores_out[s] = sc;
      }
      id = uint32_t(__builtin_amdgcn_readlane(int(id), j));
    } else {  // only the slot's own pick: the expert of rank j
      id = rank_pick_wave<N>(v, n_experts, j);
    }
    e = id;
  }
  if constexpr (TL) {
    asm volatile("" ::"v"(e));
    tl_stamp<TL>(tl, 2);
  }
  // no such expert: zero rows (cpu_kern.cpp:316-318); the folded shared expert is expert n_experts
  const bool valid = e < uint32_t(n_experts) || shared_slot;
  const size_t rsafe = size_t(valid ? e : 0u) * I + min(r0, I - RB);
  const u32x4 *gsrc = reinterpret_cast<const u32x4 *>(wg + rsafe * (36 * P));
  const u32x4 *usrc = reinterpret_cast<const u32x4 *>(wu + rsafe * (36 * P));
  // the gate rows' C chunks then the up rows' as one run of 2 C (a lane past the end reloads the last chunk): stage
  // chunk q holds gate chunk q (q < C) or up chunk q - C
  u32x4 vw[NC2];
#pragma unroll
  for (int i = 0; i < NC2; ++i) {
    const int q = min(lane + 64 * i, 2 * C - 1);
    vw[i] = __builtin_nontemporal_load(q < C ? gsrc + q : usrc + (q - C));
  }
  // the activation row into LDS (a thread past the end rewrites the last chunk with its own value; RAW: prepared
  // here from the raw row), then the weights into the wavefront's stage, with no branch between loads and stores so
  // that no load is sunk into a conditional block behind the others' wait
  if (RAW) {
    const int xch = xdt == LMOE_F32 ? 16 * P : 8 * P;
#pragma unroll
    for (int i = 0; i < XRR; ++i)
      if (int(threadIdx.x) + NT * i < xch) xraw[threadIdx.x + NT * i] = xr4[i];
    __syncthreads();
  }
  if (RAW) {  // the pair dwords, then each unit's two sums and two pads (no thread mixes the two kinds)
    const _Float16 *xh = reinterpret_cast<const _Float16 *>(xraw);
    const uint16_t *xb = reinterpret_cast<const uint16_t *>(xraw);
    const float *xf = reinterpret_cast<const float *>(xraw);
    uint32_t *xd = reinterpret_cast<uint32_t *>(xl);
    auto go = [&](auto ld) {
      for (int idx = threadIdx.x; idx < P * 32; idx += NT) {
        const int pu = idx >> 5, dw = idx & 31;
        xd[pu * XS + dw] = prep_dword<TQ>(ld, pu, dw);
      }
      for (int idx = threadIdx.x; idx < P * 4; idx += NT) {
        const int pu = idx >> 2, dw = 32 + (idx & 3);
        xd[pu * XS + dw] = prep_dword<TQ>(ld, pu, dw);
      }
    };
    if (xdt == LMOE_F16)
      go([&](int i) { return float(xh[i]); });
    else if (xdt == LMOE_BF16)
      go([&](int i) { return bf16_to_f32(xb[i]); });
    else
      go([&](int i) { return xf[i]; });
  } else {
#pragma unroll
    for (int i = 0; i < XPT; ++i) xl[min(int(threadIdx.x) + NT * i, XC - 1)] = xc[i];
  }
  __syncthreads();
  // this lane's activation unit out of LDS while the weights are still on their way, then the weights into the stage
  uint32_t xv[32];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const u32x4 q = xl[9 * p + i];
    xv[4 * i] = q.x;
    xv[4 * i + 1] = q.y;
    xv[4 * i + 2] = q.z;
    xv[4 * i + 3] = q.w;
  }
  // the two half-unit sums; __uint_as_float, not __builtin_bit_cast: this compiler lowers a bit cast of an
  // ext_vector element lvalue (qs.y) to element 0
  const u32x4 qs = xl[9 * p + 8];
  const float sx0 = __uint_as_float(qs.x), sx1 = __uint_as_float(qs.y);
  u32x4 *st4 = reinterpret_cast<u32x4 *>(stage);
#pragma unroll
  for (int i = 0; i < NC2; ++i) st4[min(lane + 64 * i, 2 * C - 1)] = vw[i];
  __builtin_amdgcn_wave_barrier();
  tl_stamp<TL>(tl, 3);
  if (r0 >= I) return;
  if (!valid) {
    if (lane < RB) {
      const int n = r0 + lane;
      if (h) h[size_t(s) * I + n] = 0.0f;
      if (hprep) {
        int dw, half;
        xslot(n & 63, td == LMOE_Q4_K ? 32 : 16, &dw, &half);
        reinterpret_cast<_Float16 *>(hprep + (size_t(s) * (I / 64) + (n >> 6)) * XS + dw)[half] = _Float16(0.0f);
      }
    }
    return;
  }
  float pg[RG], pu[RG];
#pragma unroll
  for (int i = 0; i < RG; ++i) {
    const int rr = g + G * i;
    pg[i] = row_unit_dot_r<TQ>(stage + rr * 9 * P, p, xv, sx0, sx1);
    pu[i] = row_unit_dot_r<TQ>(stage + (RB + rr) * 9 * P, p, xv, sx0, sx1);
  }
#pragma unroll
  for (int i = 0; i < RG; ++i) {
    pg[i] = group_sum<P>(pg[i]);
    pu[i] = group_sum<P>(pu[i]);
  }
  if (p == 0) {
#pragma unroll
    for (int i = 0; i < RG; ++i) {
      const int n = r0 + g + G * i;
      const float hv = silu_mul(pg[i], pu[i]);
      if (h) h[size_t(s) * I + n] = hv;
      if (hprep) {
        int dw, half;
        xslot(n & 63, td == LMOE_Q4_K ? 32 : 16, &dw, &half);
        reinterpret_cast<_Float16 *>(hprep + (size_t(s) * (I / 64) + (n >> 6)) * XS + dw)[half] = _Float16(hv);
      }
    }
  }
  tl_stamp<TL>(tl, 4);
}

// ---- down + combine -------------------------------------------------------------------------------------------
//
// Grid (H / (4 NW), T). Block (bx, t) stages the k h rows of token t as prepared units (copied from hprep, sums
// derived when has_sums is 0; or rearranged from fp32 h), then wavefront w takes output rows [(bx NW + w) 4, +4)
// of all k experts of token t, adds them weighted by scores[t] (1 when scores is null), then the gated
// shared-expert row and the residual, and writes out[t]. When k 9 P <= 64 NC the weight chunks are fetched into
// registers before the h staging; otherwise after it.
template <int TD, int RB, int NC, int NW, bool HP, bool PRE>
__global__ void __launch_bounds__(64 * NW, 3)
    k_down_combine(const uint32_t *hprep, int has_sums, const float *h, const uint32_t *ids, const float *scores,
                   int k, const uint8_t *wd, int n_experts, int I, int H, const float *shared, const float *gate,
                   int gate_stride, const void *residual, int rdt, void *out, int odt) {
  const int P = I / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = blockIdx.y;
  const int n0 = (blockIdx.x * NW + wave) * RB;
  extern __shared__ u32x4 lds4[];
  uint32_t *hx = reinterpret_cast<uint32_t *>(lds4);          // k * P * XS
  uint32_t *eid = hx + k * P * XS;                             // 32
  float *esc = reinterpret_cast<float *>(eid + 32);           // 32
  uint32_t *region = reinterpret_cast<uint32_t *>(esc + 32);
  const int stage_dw = k * RB * 9 * P;
  const int hraw_dw = hprep ? 0 : k * I;
  uint32_t *stage = region + wave * stage_dw;
  const int red_ld = k * P + 1;
  float *red = reinterpret_cast<float *>(region + max(NW * stage_dw, hraw_dw)) + wave * (RB * red_ld);

  const size_t rowb = size_t(36) * P;
  const int C = RB * 9 * P / 4;  // 16-byte chunks of RB rows
  const bool rows_ok = n0 < H;
  // Memory order of the prologue: the token's ids and scores (one a lane), the first 8 16-byte chunks a thread of
  // its prepared h rows, then the weights, whose addresses need only the ids. No load is predicated (clamped
  // indices; expert 0 stands in for an id past the experts, the last row block for a wavefront past H), so each
  // group issues back to back and the h stores to LDS wait only for the h loads.
  const uint32_t *tid_ids = ids + size_t(t) * k;
  const int kl = min(lane, k - 1);
  const uint32_t my_id = tid_ids[kl];
  const float sc_ld = (scores ? scores + size_t(t) * k : reinterpret_cast<const float *>(tid_ids))[kl];
  const float my_sc = scores ? sc_ld : 1.0f;  // read by lane exchange in the dot loop, once the weights are in
  const int nthr = 64 * NW;
  const int hn = HP ? k * P * XS / 4 : 0;
  const u32x4 *hsrc = reinterpret_cast<const u32x4 *>(hprep + size_t(t) * k * P * XS);
  u32x4 hv[8];
  if (HP) {
#pragma unroll
    for (int j = 0; j < 8; ++j) hv[j] = hsrc[min(int(threadIdx.x) + j * nthr, hn - 1)];
  }
  u32x4 v[NC];
  if (PRE) {
    const size_t nsafe = size_t(min(n0, H - RB));
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = min(lane + 64 * i, k * C - 1);
      const int j = c / C, cc = c - j * C;
      uint32_t e = uint32_t(__shfl(int(my_id), j, 64));
      e = e < uint32_t(n_experts) ? e : 0u;
      v[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(wd + (size_t(e) * H + nsafe) * rowb) + cc);
    }
  }
  if (threadIdx.x < k) {  // wavefront 0, lane = threadIdx.x < k <= 32
    eid[threadIdx.x] = my_id;
  }
  if (HP) {
    u32x4 *hx4 = reinterpret_cast<u32x4 *>(hx);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (int(threadIdx.x) + j * nthr < hn) hx4[threadIdx.x + j * nthr] = hv[j];
    if (hn > 8 * nthr)
      copy_to_lds(hsrc + 8 * nthr, hx4 + 8 * nthr, 4 * (hn - 8 * nthr), threadIdx.x, nthr);
    __syncthreads();
    if (!has_sums) {
      sums_in_lds<TD>(hx, k * P, threadIdx.x, nthr);
      __syncthreads();
    }
  } else {
    copy_to_lds(h + size_t(t) * k * I, region, k * I, threadIdx.x, nthr);
    __syncthreads();
    for (int j = 0; j < k; ++j) prep_in_lds<TD>(region + j * I, LMOE_F32, P, hx + j * P * XS, threadIdx.x, nthr);
    __syncthreads();
  }
  if (!rows_ok) return;

  u32x4 *st4 = reinterpret_cast<u32x4 *>(stage);
  if (PRE) {
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
#pragma unroll 2
  for (int u0 = 0; u0 < U; u0 += 64) {  // uniform trip count: the score exchange runs with every lane active
    const int u = min(u0 + lane, U - 1);
    const int j = u / (RB * P), rem = u - j * (RB * P), row = rem / P, p = rem - row * P;
    const float sc = __shfl(my_sc, j, 64);
    if (u0 + lane < U) {
      float part = 0.0f;
      if (eid[j] < uint32_t(n_experts))
        part = sc * row_unit_dot<TD>(stage + (j * RB + row) * 9 * P, p, hx + (j * P + p) * XS);
      red[row * red_ld + j * P + p] = part;
    }
  }
  __builtin_amdgcn_wave_barrier();

  constexpr int LPR = 64 / RB;
  const int rr = lane / LPR, sub = lane % LPR;
  float acc = 0.0f;
  for (int i = sub; i < k * P; i += LPR) acc += red[rr * red_ld + i];
  acc = sum16(acc);
  if (LPR == 32) acc += lane_xor16(acc);
  const int n = n0 + rr;
  if (sub == 0 && n < H) {
    const size_t o = size_t(t) * H + n;
    if (shared) acc += sigmoidf_(gate[size_t(t) * gate_stride]) * shared[o];
    if (residual) acc += load_elt(residual, o, rdt);
    store_elt(out, o, acc, odt);
  }
}

// ---- down + combine with the h units in registers ---------------------------------------------------------------
//
// For prepared h and k P <= 64 NU (k experts of P = I / 64 units; NU = 1 or 2 units a lane), P even. KS = 1: grid
// (H / (4 RB), T), four independent wavefronts a workgroup (no barrier); wavefront w of block (bx, t) takes output
// rows [(4 bx + w) RB, +RB) of token t. KS = 2 (the host's default where k >= 2): grid (H / (2 RB), T), two
// wavefronts a row pair over half of the experts each, their sums met through LDS after one barrier (below). The
// rest is written for KS = 1. Lane l holds h units u = l, l + 64 (u = j P + p: expert j, unit p) in
// registers and their half-unit sums, computed there while the weights are in flight. The wavefront's RB rows of all
// k experts (k RB 36 P bytes) come in with 16-byte loads, go to its own LDS region, and each lane dots its units with
// the RB rows of its expert (a 36-byte unit read a dot), weighted by the router score; the rows' sums over the
// wavefront finish on DPP / permlane swaps, then the gated shared-expert row and the residual are added. Memory order:
// h units, ids and scores (one a lane), then the weights, whose addresses need only the ids; no load is predicated
// (clamped indices; expert 0 stands in for an id past the experts, with a zero weight).
template <int TD, int NU, int NCW, int KS = 1, int HL = 0, bool TL = false, int NWG = 4>
__global__ void __launch_bounds__(64 * NWG)
    k_down_xr(const uint32_t *hprep, const uint32_t *ids, const float *scores, int k, const uint8_t *wd,
              int n_experts, int I, int H, const float *shared, const float *gate, int gate_stride,
              const void *residual, int rdt, void *out, int odt, unsigned long long *tl) {
  constexpr int RB = 2;
  tl_stamp<TL>(tl, 0);
  static_assert(KS == 1 || KS == 2, "experts split over 1 or 2 wavefronts");
  static_assert(NWG == 4 || (NWG == 8 && KS == 2), "4 wavefronts a workgroup, or 8 (4 row pairs) with KS = 2");
  // KS = 2: wavefronts 2 g and 2 g + 1 share rows [(2 bx + g) RB, +RB), wavefront 2 g + q over experts
  // [q kh, q kh + kh) (kh = ceil(k / 2); k >= 2, so both shares hold experts), and the second share's row sums are
  // added to the first's through LDS
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = KS > 1 ? wave % KS : 0;
  const int kh = KS > 1 ? (k + KS - 1) / KS : k;
  const int j0 = q * kh, kj = KS > 1 ? min(kh, k - j0) : k;  // this wavefront's experts [j0, j0 + kj)
  const int P = I / 64, U = kj * P;
  const int CJ = RB * 9 * P / 4, CW = kj * CJ;  // 16-byte chunks of one expert's RB rows, of this wavefront's
  const int t = blockIdx.y;
  const int n0 = (blockIdx.x * (NWG / KS) + wave / KS) * RB;
  extern __shared__ u32x4 lds4[];
  uint32_t *stage = reinterpret_cast<uint32_t *>(lds4) + wave * (kh * CJ * 4);
  // HL > 0: the wavefront's h chunks through LDS, after the NWG stages: 64 HL chunks a wavefront. KS = 2: the NWG / 2
  // wavefronts over the same experts (one a row pair each) share one copy, each loading every (NWG / 2)-th 64-chunk
  // block of it
  constexpr bool SH = KS == 2 && HL > 0;
  constexpr int HW = SH ? NWG / 2 : 1;         // wavefronts sharing one copy
  constexpr int HLS = (HL + HW - 1) / HW;      // h loads a lane
  const int hblk = SH ? wave / 2 : 0;          // this wavefront's blocks: HW i + hblk
  u32x4 *hst = lds4 + NWG * kh * CJ + (SH ? q : wave) * 64 * HL;

  // 1. the token's ids and scores (lane j < k holds expert j's), then the h units. The empty asm with a memory
  // clobber keeps the compiler from sinking these loads below the weights' (the count of outstanding loads is in
  // order, so the weight addresses then wait only for the ids and scores, and the h sums only for the h units).
  // HL = 0: lane l loads its own units' 8 value chunks (8 NU loads); HL > 0: the wavefront's 8 U chunks as one run of
  // HL loads a lane (ceil(8 U / 64): 6 instead of 8 at 48 units), unit-ordered into LDS below
  const int kl = min(lane, k - 1);
  const uint32_t my_id = ids[size_t(t) * k + kl];
  const float sc_ld = (scores ? scores + size_t(t) * k : reinterpret_cast<const float *>(ids))[kl];
  const float my_sc = scores ? sc_ld : 1.0f;
  const u32x4 *hb = reinterpret_cast<const u32x4 *>(hprep + (size_t(t) * k + j0) * P * XS);
  u32x4 hq[NU][8];
  u32x4 hl[HL > 0 ? HLS : 1];
  if constexpr (HL > 0) {
#pragma unroll
    for (int i = 0; i < HLS; ++i) {
      const int qc = min(lane + 64 * (HW * i + hblk), 8 * U - 1);
      hl[i] = hb[(qc >> 3) * 9 + (qc & 7)];
    }
  } else {
#pragma unroll
    for (int a = 0; a < NU; ++a) {
      const int u = min(lane + 64 * a, U - 1);
#pragma unroll
      for (int i = 0; i < 8; ++i) hq[a][i] = hb[u * 9 + i];
    }
  }
  // the epilogue's inputs: the residual's dword holding this lane's element, the shared expert's row element and its
  // gate logit (a null pointer reads the first id instead, ignored at the end). Loaded with no branch, so that no
  // counted wait moves, and early, so that the end waits on no round trip of its own: for Q4_K (cfg5's shape, 16
  // wavefronts a CU) before the weights, else after them (measured on one box, µs a layer: Q4_K 22.69 after against
  // 22.45 before; Q4_0 at cfg2 13.64 after against 13.73 before)
  constexpr bool kEpiFirst = TD == LMOE_Q4_K;
  const size_t o_pf = size_t(t) * H + min(n0, H - RB) + min(lane, RB - 1);
  uint32_t res_w;
  float sh_pf, gate_pf;
  auto load_epilogue = [&] {
    const size_t r_off = rdt == LMOE_F32 ? o_pf * 4 : (o_pf * 2) & ~size_t(3);
    res_w = *reinterpret_cast<const uint32_t *>(residual ? static_cast<const char *>(residual) + r_off
                                                         : reinterpret_cast<const char *>(ids));
    sh_pf = shared ? shared[o_pf] : reinterpret_cast<const float *>(ids)[0];
    gate_pf = shared ? gate[size_t(t) * gate_stride] : reinterpret_cast<const float *>(ids)[0];
  };
  if constexpr (kEpiFirst) load_epilogue();
  asm volatile("" ::: "memory");
  // the ids through an empty asm after that one, so that the weight addresses' lane shuffles (no memory access, free
  // to move) cannot be hoisted above the h loads and make them wait for the ids
  const uint32_t my_id_l = opaque(my_id);
  if constexpr (TL) tl_stamp<TL>(tl, 1);
  // 2. the weights: chunk c of expert j0 + j's block at rows [n0, n0 + RB)
  const size_t rowb = size_t(36) * P, nsafe = size_t(min(n0, H - RB));
  u32x4 w[NCW];
#pragma unroll
  for (int i = 0; i < NCW; ++i) {
    const int c = min(lane + 64 * i, CW - 1);
    const int j = c / CJ, cc = c - j * CJ;
    uint32_t e = uint32_t(__shfl(int(my_id_l), j0 + j, 64));
    e = e < uint32_t(n_experts) ? e : 0u;
    w[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(wd + (size_t(e) * H + nsafe) * rowb) + cc);
  }
  asm volatile("" ::: "memory");
  if constexpr (!kEpiFirst) load_epilogue();
  // 3. (HL > 0: the h chunks into LDS, chunk c of unit u at 8 u + (c ^ ((u >> 1) & 7)), so that neither the run's
  // writes nor each lane's reads of its own unit meet twice in a bank group; then each lane's units back), each
  // unit's expert, weight (0 past the units or the experts) and half-unit sums
  if constexpr (HL > 0) {
#pragma unroll
    for (int i = 0; i < HLS; ++i) {  // a lane past the end rewrites the last chunk (the same value)
      const int qc = min(lane + 64 * (HW * i + hblk), 8 * U - 1), u = qc >> 3;
      hst[8 * u + ((qc & 7) ^ ((u >> 1) & 7))] = hl[i];
    }
    if constexpr (SH)
      __syncthreads();
    else
      __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int a = 0; a < NU; ++a) {
      const int u = min(lane + 64 * a, U - 1);
#pragma unroll
      for (int i = 0; i < 8; ++i) hq[a][i] = hst[8 * u + (i ^ ((u >> 1) & 7))];
    }
  }
  int ja[NU], pa[NU];
  float fa[NU], s0[NU], s1[NU];
  uint32_t xv[NU][32];
  const h2_t one2 = {_Float16(1.0f), _Float16(1.0f)};
#pragma unroll
  for (int a = 0; a < NU; ++a) {
    const int u = lane + 64 * a, uc = min(u, U - 1);
    ja[a] = uc / P;
    pa[a] = uc - ja[a] * P;
    const uint32_t e = uint32_t(__shfl(int(my_id_l), j0 + ja[a], 64));
    const float sj = __shfl(my_sc, j0 + ja[a], 64);
    fa[a] = (u < U && e < uint32_t(n_experts)) ? sj : 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      xv[a][4 * i] = hq[a][i].x;
      xv[a][4 * i + 1] = hq[a][i].y;
      xv[a][4 * i + 2] = hq[a][i].z;
      xv[a][4 * i + 3] = hq[a][i].w;
    }
    float x0 = 0.0f, x1 = 0.0f;  // a unit's first / last 32 values: dwords 0..15 / 16..31 (Q4_0), even / odd (Q4_K)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t d0 = TD == LMOE_Q4_K ? xv[a][2 * i] : xv[a][i];
      const uint32_t d1 = TD == LMOE_Q4_K ? xv[a][2 * i + 1] : xv[a][16 + i];
      x0 = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, d0), one2, x0, false);
      x1 = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, d1), one2, x1, false);
    }
    s0[a] = x0;
    s1[a] = x1;
  }
  // 4. the weights into the wavefront's stage (no branch between loads and stores)
  u32x4 *st4 = reinterpret_cast<u32x4 *>(stage);
#pragma unroll
  for (int i = 0; i < NCW; ++i) st4[min(lane + 64 * i, CW - 1)] = w[i];
  __builtin_amdgcn_wave_barrier();
  tl_stamp<TL>(tl, 3);
  if (KS == 1 && n0 >= H) return;  // (KS == 2: the host launches exactly H / 4 workgroups, every row in range)
  // 5. dots
  float acc[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) acc[r] = 0.0f;
#pragma unroll
  for (int a = 0; a < NU; ++a)
#pragma unroll
    for (int r = 0; r < RB; ++r)
      acc[r] = fmaf(fa[a], row_unit_dot_r<TD>(stage + (ja[a] * RB + r) * 9 * P, pa[a], xv[a], s0[a], s1[a]), acc[r]);
  // 6. the rows' sums (KS = 2: the second share's through LDS into the first's), then shared expert and residual
#pragma unroll
  for (int r = 0; r < RB; ++r) acc[r] = wave_sum(acc[r]);
  if (KS == 2) {
    __shared__ float part[NWG * RB];  // [wavefront][row]
    if (q == 1 && lane < RB) part[wave * RB + lane] = lane == 0 ? acc[0] : acc[1];
    __syncthreads();
    if (q == 1) return;
#pragma unroll
    for (int r = 0; r < RB; ++r) acc[r] += part[(wave + 1) * RB + r];
  }
  if (lane < RB) {
    float v = acc[0];
#pragma unroll
    for (int r = 1; r < RB; ++r) v = lane == r ? acc[r] : v;
    const size_t o = size_t(t) * H + n0 + lane;
    if (shared) v += sigmoidf_(gate_pf) * sh_pf;
    if (residual) {
      const uint32_t hb16 = (o & 1) ? res_w >> 16 : res_w & 0xFFFFu;
      v += rdt == LMOE_F32   ? __uint_as_float(res_w)
           : rdt == LMOE_F16 ? float(__builtin_bit_cast(_Float16, uint16_t(hb16)))
                             : __uint_as_float(hb16 << 16);
    }
    store_elt(out, o, v, odt);
  }
  tl_stamp<TL>(tl, 4);
}

// ---- host dispatch ----------------------------------------------------------------------------------------------

// ---- the decode chain on runs of equal slots (one slot a row) ----------------------------------------------------
//
// The reference's run kernels (gguf_experts.py:600-607, gguf_cuda.py:33-152): rows of one slot each, best sorted by
// slot, go through windows of up to TR rows; a wavefront loads its weight rows once a run of equal slots in the
// window and reuses them for every row of the run. Per row the arithmetic is the chain's own (the same prepared
// activation units, unit dots, partial layout and reduction tree as k_gate_up / k_down_combine at the same RB), so
// the outputs are meant to be bit-equal to the chain's; the host checks that once a shape before using them.
// Latency is what bounds both kernels (a few KB of weights a wavefront a run), so every round trip is overlapped:
// the window's slot ids are read once, the first run's weights are in flight while the window's rows are prepared,
// and each run's successor is fetched into registers while the run computes.

// Rows [row0, row0 + nr) of x (64 P elements each, dtype dt, 16-byte aligned) as prepared units of block type TQ
// into dst [nr][P XS]: the f16 values go straight from 16-byte global loads to their (dword, half) places, then the
// half sums are read back from them in element order, which gives prep_dword's bits without staging the raw rows.
// Ends with a workgroup barrier.
template <int TQ>
__device__ __forceinline__ void prep_rows(const void *x, int dt, size_t row0, int nr, int P, uint32_t *dst, int tid,
                                          int nthr) {
  constexpr int HS = TQ == LMOE_Q4_K ? 32 : 16;
  const int esz = dt == LMOE_F32 ? 4 : 2, per = 16 / esz;  // elements a 16-byte chunk
  const int cpr = 64 * P / per;                              // chunks a row
  const int n = nr * cpr;
  const u32x4 *src = reinterpret_cast<const u32x4 *>(static_cast<const char *>(x) + row0 * 64 * P * esz);
  for (int b = tid; b < n; b += 8 * nthr) {
    u32x4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = src[min(b + j * nthr, n - 1)];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int c = b + j * nthr;
      if (c < n) {
        const int r = c / cpr, i0 = (c - r * cpr) * per;
        _Float16 *row = reinterpret_cast<_Float16 *>(dst + r * P * XS);
        const uint32_t w[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
        for (int k = 0; k < per; ++k) {
          float f;
          if (dt == LMOE_F32) {
            f = __uint_as_float(w[k]);
          } else {
            const uint16_t bits = uint16_t(w[k >> 1] >> (16 * (k & 1)));
            f = dt == LMOE_F16 ? float(__builtin_bit_cast(_Float16, bits)) : bf16_to_f32(bits);
          }
          const int i = i0 + k;
          int dw, half;
          xslot(i & 63, HS, &dw, &half);
          row[2 * ((i >> 6) * XS + dw) + half] = _Float16(f);
        }
      }
    }
  }
  for (int q = tid; q < nr * P; q += nthr) {
    dst[q * XS + 34] = 0u;
    dst[q * XS + 35] = 0u;
  }
  __syncthreads();
  for (int hu = tid; hu < nr * P * 2; hu += nthr) {
    const int q = hu >> 1, half = hu & 1;
    const _Float16 *u = reinterpret_cast<const _Float16 *>(dst + q * XS);
    float s = 0.0f;
    for (int j = 0; j < 32; ++j) {
      int dw, hf;
      xslot(32 * half + j, HS, &dw, &hf);
      s += float(u[2 * dw + hf]);
    }
    dst[q * XS + 32 + half] = __builtin_bit_cast(uint32_t, s);
  }
  __syncthreads();
}

constexpr int kRunQ = 4;  // rows of a run whose unit dots go out in one loop

// Gate/up: grid (ceil(I / (RB NW)), ceil(n / TR)); wavefront w of block (bx, y) takes gate and up rows
// [(bx NW + w) RB, +RB) for rows [y TR, +TR) of x. LDS: the window's prepared rows (gate's, then up's when the types
// differ), its slot ids, each wavefront's 2 RB staged weight rows, then each wavefront's partials of kRunQ rows.
// NC >= ceil(RB 9 P / 4 / 64) 16-byte chunks a lane a matrix.
template <int TG, int TU, int RB, int NW, int NC>
__global__ void __launch_bounds__(64 * NW)
    k_gate_up_runs(const void *x, int xdt, const uint32_t *slots, int n, int tr, const uint8_t *wg,
                   const uint8_t *wu, int n_experts, int I, int P, float *h) {
  constexpr bool SAME = TG == TU;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r0 = (blockIdx.x * NW + wave) * RB;
  const int e0 = blockIdx.y * tr, ne = min(tr, n - e0);
  const int stage_dw = 2 * RB * 9 * P, U = 2 * RB * P, RL = 2 * RB * (P + 1);
  extern __shared__ u32x4 lds4[];
  uint32_t *xg = reinterpret_cast<uint32_t *>(lds4);
  uint32_t *xu = SAME ? xg : xg + tr * P * XS;
  uint32_t *sl = xu + tr * P * XS;
  uint32_t *stage = sl + ((tr + 3) & ~3) + wave * stage_dw;
  float *red = reinterpret_cast<float *>(sl + ((tr + 3) & ~3) + NW * stage_dw) + wave * kRunQ * RL;

  // the first run's rows into registers, unpredicated (a wavefront past the rows reads the last row block, an id
  // past the experts expert 0's), while the window is prepared
  const int C = RB * 9 * P / 4;
  const size_t rowb = size_t(36) * P;
  const int rs = min(r0, I - RB);
  u32x4 vg[NC], vu[NC];
  auto fetch = [&](uint32_t e) {
    const size_t base = (size_t(e < uint32_t(n_experts) ? e : 0u) * I + rs) * rowb;
    const u32x4 *gs = reinterpret_cast<const u32x4 *>(wg + base);
    const u32x4 *us = reinterpret_cast<const u32x4 *>(wu + base);
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = min(lane + 64 * i, C - 1);
      vg[i] = __builtin_nontemporal_load(gs + c);
      vu[i] = __builtin_nontemporal_load(us + c);
    }
  };
  fetch(slots[e0]);
  if (int(threadIdx.x) < ne) sl[threadIdx.x] = slots[e0 + threadIdx.x];
  prep_rows<TG>(x, xdt, e0, ne, P, xg, threadIdx.x, 64 * NW);
  if (!SAME) prep_rows<TU>(x, xdt, e0, ne, P, xu, threadIdx.x, 64 * NW);
  if (r0 >= I) return;

  u32x4 *st4 = reinterpret_cast<u32x4 *>(stage);
  constexpr int LPR = 64 / (2 * RB);
  const int rr = lane / LPR, sub = lane % LPR;
  for (int r = 0; r < ne;) {
    const uint32_t e = sl[r];
    int r1 = r + 1;  // the run: rows [r, r1) of slot e
    while (r1 < ne && sl[r1] == e) ++r1;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = lane + 64 * i;
      if (c < C) {
        st4[c] = vg[i];
        st4[C + c] = vu[i];
      }
    }
    if (r1 < ne) fetch(sl[r1]);  // the next run's rows, in flight during this one
    __builtin_amdgcn_wave_barrier();
    if (e >= uint32_t(n_experts)) {  // no such expert: zero rows (cpu_kern.cpp:316-318)
      for (int q = r; q < r1; ++q)
        if (lane < RB) h[size_t(e0 + q) * I + r0 + lane] = 0.0f;
      r = r1;
      continue;
    }
    for (int q0 = r; q0 < r1; q0 += kRunQ) {
      const int nq = min(kRunQ, r1 - q0);
#pragma unroll 2
      for (int v = lane; v < nq * U; v += 64) {
        const int q = v / U, u = v - q * U;
        const int row = u / P, p = u - row * P;
        float part;
        if (row < RB)
          part = row_unit_dot<TG>(stage + row * 9 * P, p, xg + ((q0 + q) * P + p) * XS);
        else
          part = row_unit_dot<TU>(stage + row * 9 * P, p, xu + ((q0 + q) * P + p) * XS);
        red[q * RL + row * (P + 1) + p] = part;
      }
      __builtin_amdgcn_wave_barrier();
      for (int q = 0; q < nq; ++q) {
        float acc = 0.0f;
        for (int p = sub; p < P; p += LPR) acc += red[q * RL + rr * (P + 1) + p];
        acc = LPR == 8 ? sum8(acc) : sum16(acc);
        const float up = lane_xor32(acc);
        if (rr < RB && sub == 0) h[size_t(e0 + q0 + q) * I + r0 + rr] = silu_mul(acc, up);
      }
      __builtin_amdgcn_wave_barrier();
    }
    r = r1;
  }
}

// Down of the same windows, unweighted: grid (ceil(H / (RB NW)), ceil(n / TR)); wavefront w of block (bx, y) takes
// output rows [(bx NW + w) RB, +RB) for h rows [y TR, +TR). LDS: the window's prepared h rows, its slot ids, each
// wavefront's RB staged weight rows, then each wavefront's partials of kRunQ rows.
template <int TD, int RB, int NW, int NC>
__global__ void __launch_bounds__(64 * NW)
    k_down_runs(const float *h, const uint32_t *slots, int n, int tr, const uint8_t *wd, int n_experts, int I, int H,
                void *out, int odt) {
  const int P = I / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = (blockIdx.x * NW + wave) * RB;
  const int e0 = blockIdx.y * tr, ne = min(tr, n - e0);
  const int stage_dw = RB * 9 * P, red_ld = P + 1, U = RB * P, RL = RB * red_ld;
  extern __shared__ u32x4 lds4[];
  uint32_t *hx = reinterpret_cast<uint32_t *>(lds4);
  uint32_t *sl = hx + tr * P * XS;
  uint32_t *stage = sl + ((tr + 3) & ~3) + wave * stage_dw;
  float *red = reinterpret_cast<float *>(sl + ((tr + 3) & ~3) + NW * stage_dw) + wave * kRunQ * RL;

  const size_t rowb = size_t(36) * P;
  const int C = RB * 9 * P / 4;
  const int ns = min(n0, H - RB);
  u32x4 v[NC];
  auto fetch = [&](uint32_t e) {
    const u32x4 *src =
        reinterpret_cast<const u32x4 *>(wd + (size_t(e < uint32_t(n_experts) ? e : 0u) * H + ns) * rowb);
#pragma unroll
    for (int i = 0; i < NC; ++i) v[i] = __builtin_nontemporal_load(src + min(lane + 64 * i, C - 1));
  };
  fetch(slots[e0]);
  if (int(threadIdx.x) < ne) sl[threadIdx.x] = slots[e0 + threadIdx.x];
  prep_rows<TD>(h, LMOE_F32, e0, ne, P, hx, threadIdx.x, 64 * NW);
  if (n0 >= H) return;

  u32x4 *st4 = reinterpret_cast<u32x4 *>(stage);
  constexpr int LPR = 64 / RB;
  const int rr = lane / LPR, sub = lane % LPR;
  for (int r = 0; r < ne;) {
    const uint32_t e = sl[r];
    int r1 = r + 1;
    while (r1 < ne && sl[r1] == e) ++r1;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < NC; ++i)
      if (lane + 64 * i < C) st4[lane + 64 * i] = v[i];
    if (r1 < ne) fetch(sl[r1]);
    __builtin_amdgcn_wave_barrier();
    if (e >= uint32_t(n_experts)) {
      for (int q = r; q < r1; ++q)
        if (sub == 0) store_elt(out, size_t(e0 + q) * H + n0 + rr, 0.0f, odt);
      r = r1;
      continue;
    }
    for (int q0 = r; q0 < r1; q0 += kRunQ) {
      const int nq = min(kRunQ, r1 - q0);
#pragma unroll 2
      for (int w = lane; w < nq * U; w += 64) {
        const int q = w / U, u = w - q * U;
        const int row = u / P, p = u - row * P;
        red[q * RL + row * red_ld + p] = row_unit_dot<TD>(stage + row * 9 * P, p, hx + ((q0 + q) * P + p) * XS);
      }
      __builtin_amdgcn_wave_barrier();
      for (int q = 0; q < nq; ++q) {
        float acc = 0.0f;
        for (int i = sub; i < P; i += LPR) acc += red[q * RL + rr * red_ld + i];
        acc = sum16(acc);
        if (LPR == 32) acc += lane_xor16(acc);
        if (sub == 0) store_elt(out, size_t(e0 + q0 + q) * H + n0 + rr, acc, odt);
      }
      __builtin_amdgcn_wave_barrier();
    }
    r = r1;
  }
}

// ---- run kernels on prepared rows: per row the register-resident chain's arithmetic ------------------------------
//
// The run kernels above follow k_gate_up / k_down_combine. These two follow the kernels the drop-in chain takes when
// the shapes allow it: k_gate_up_xr with slots given, and k_down_xr at one slot a row, unweighted. Per row they use
// the same staged weight rows, the same activation unit in the same lane, the same unit dots and the same cross-lane
// sums, so h, its prepared rows and the outputs are meant to be bit-equal to that chain's; the host checks that once
// a shape before it uses them.
//
// Gate/up: grid (ceil(I / 8), ceil(n / tr)), 256 threads; wavefront w of block (bx, y) takes gate and up rows
// [(4 bx + w) 2, +2) for the prepared rows [y tr, +tr) of x, lane (g, p) unit p of row g as in k_gate_up_xr. LDS:
// the window's prepared rows (copied as they are), its slot ids, each wavefront's 2 gate + 2 up staged rows.
template <int TQ, int P>
__global__ void __launch_bounds__(256)
    k_gate_up_runs_xr(const uint32_t *xprep, const uint32_t *slots, int n, int tr, const uint8_t *wg,
                      const uint8_t *wu, int n_experts, int I, float *h, uint32_t *hprep, int td) {
  static_assert(P == 32 || P == 64, "32 or 64 units a row");
  constexpr int RB = 2, G = 64 / P, RG = RB / G;
  constexpr int C = RB * 9 * P / 4;  // 16-byte chunks of RB rows of one matrix
  constexpr int NC2 = (2 * C + 63) / 64;  // of both matrices' rows, a lane (one run, as in k_gate_up_xr)
  constexpr int STAGE = 2 * RB * 9 * P;  // dwords a wavefront
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r0 = (blockIdx.x * 4 + wave) * RB;
  const int e0 = blockIdx.y * tr, ne = min(tr, n - e0);
  const int g = lane / P, p = lane % P;
  extern __shared__ u32x4 lds4[];
  u32x4 *xw = lds4;  // 9 P chunks a row
  uint32_t *sl = reinterpret_cast<uint32_t *>(lds4 + size_t(tr) * 9 * P);
  u32x4 *st4 = reinterpret_cast<u32x4 *>(sl + ((tr + 3) & ~3) + wave * STAGE);
  const uint32_t *stage = reinterpret_cast<const uint32_t *>(st4);

  // the first run's rows into registers (clamped, unpredicated) while the window is copied
  const int rs = min(r0, I - RB);
  u32x4 vw[NC2];
  auto fetch = [&](uint32_t e) {
    const size_t base = (size_t(e < uint32_t(n_experts) ? e : 0u) * I + rs) * (36 * P);
    const u32x4 *gs = reinterpret_cast<const u32x4 *>(wg + base);
    const u32x4 *us = reinterpret_cast<const u32x4 *>(wu + base);
#pragma unroll
    for (int i = 0; i < NC2; ++i) {
      const int q = min(lane + 64 * i, 2 * C - 1);
      vw[i] = __builtin_nontemporal_load(q < C ? gs + q : us + (q - C));
    }
  };
  fetch(slots[e0]);
  if (int(threadIdx.x) < ne) sl[threadIdx.x] = slots[e0 + threadIdx.x];
  {
    const u32x4 *src = reinterpret_cast<const u32x4 *>(xprep + size_t(e0) * P * XS);
    for (int c = threadIdx.x; c < ne * 9 * P; c += 256) xw[c] = src[c];
  }
  __syncthreads();
  if (r0 >= I) return;

  const int hs = td == LMOE_Q4_K ? 32 : 16;
  for (int r = 0; r < ne;) {
    const uint32_t e = sl[r];
    int r1 = r + 1;  // the run: rows [r, r1) of slot e
    while (r1 < ne && sl[r1] == e) ++r1;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < NC2; ++i) st4[min(lane + 64 * i, 2 * C - 1)] = vw[i];
    if (r1 < ne) fetch(sl[r1]);  // the next run's rows, in flight during this one
    __builtin_amdgcn_wave_barrier();
    const bool valid = e < uint32_t(n_experts);
    for (int q = r; q < r1; ++q) {
      const size_t row = size_t(e0 + q);
      if (!valid) {  // no such expert: zero rows, as k_gate_up_xr writes them
        if (lane < RB) {
          const int nn = r0 + lane;
          if (h) h[row * I + nn] = 0.0f;
          if (hprep) {
            int dw, half;
            xslot(nn & 63, hs, &dw, &half);
            reinterpret_cast<_Float16 *>(hprep + (row * (I / 64) + (nn >> 6)) * XS + dw)[half] = _Float16(0.0f);
          }
        }
        continue;
      }
      const u32x4 *xu4 = xw + size_t(q) * 9 * P;
      uint32_t xv[32];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const u32x4 v = xu4[9 * p + i];
        xv[4 * i] = v.x;
        xv[4 * i + 1] = v.y;
        xv[4 * i + 2] = v.z;
        xv[4 * i + 3] = v.w;
      }
      const u32x4 qs = xu4[9 * p + 8];
      const float sx0 = __uint_as_float(qs.x), sx1 = __uint_as_float(qs.y);
      float pg[RG], pu[RG];
#pragma unroll
      for (int i = 0; i < RG; ++i) {
        const int rr = g + G * i;
        pg[i] = row_unit_dot_r<TQ>(stage + rr * 9 * P, p, xv, sx0, sx1);
        pu[i] = row_unit_dot_r<TQ>(stage + (RB + rr) * 9 * P, p, xv, sx0, sx1);
      }
#pragma unroll
      for (int i = 0; i < RG; ++i) {
        pg[i] = group_sum<P>(pg[i]);
        pu[i] = group_sum<P>(pu[i]);
      }
      if (p == 0) {
#pragma unroll
        for (int i = 0; i < RG; ++i) {
          const int nn = r0 + g + G * i;
          const float hv = silu_mul(pg[i], pu[i]);
          if (h) h[row * I + nn] = hv;
          if (hprep) {
            int dw, half;
            xslot(nn & 63, hs, &dw, &half);
            reinterpret_cast<_Float16 *>(hprep + (row * (I / 64) + (nn >> 6)) * XS + dw)[half] = _Float16(hv);
          }
        }
      }
    }
    r = r1;
  }
}

// The drop-in chain's down: every slot's unweighted output from its prepared h row (without sums, as gate/up leaves
// them). A slot's P units sit on an aligned group of G lanes (G = 16, 32 or 64, at least P; two units a lane past 64),
// so SPW = 64 / G slots share a wavefront and each slot's row sums are a sum over its own group only: a slot's
// output does not depend on which slots share its wavefront, and the run kernel below repeats it bit for bit.
template <int G>
__device__ __forceinline__ float slot_sum(float v) {
  static_assert(G == 16 || G == 32 || G == 64, "a group of 16, 32 or 64 lanes");
  if (G == 64) return wave_sum(v);
  v = sum16(v);
  return G == 32 ? v + lane_xor16(v) : v;
}

// k_down_xr's half sums of an h unit held as 32 f16 pair dwords: dwords 0..15 / 16..31 (Q4_0), even / odd (Q4_K)
template <int TD>
__device__ __forceinline__ void h_unit_sums(const uint32_t *xv, float *x0, float *x1) {
  const h2_t one2 = {_Float16(1.0f), _Float16(1.0f)};
  float a = 0.0f, b = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t d0 = TD == LMOE_Q4_K ? xv[2 * i] : xv[i];
    const uint32_t d1 = TD == LMOE_Q4_K ? xv[2 * i + 1] : xv[16 + i];
    a = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, d0), one2, a, false);
    b = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, d1), one2, b, false);
  }
  *x0 = a;
  *x1 = b;
}

__device__ __forceinline__ void unpack_unit(const u32x4 *q, uint32_t *xv) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const u32x4 v = q[i];
    xv[4 * i] = v.x;
    xv[4 * i + 1] = v.y;
    xv[4 * i + 2] = v.z;
    xv[4 * i + 3] = v.w;
  }
}

// Grid (H / 8, ceil(n / SPW)), 256 threads; wavefront w of block (bx, y) takes output rows [(4 bx + w) 2, +2) of
// slots [y SPW, +SPW). Memory order as k_down_xr's: the slot ids and h units, then the weights (their addresses need
// only the ids), the half sums while they are in flight; no load is predicated (clamped indices; expert 0 stands in
// for an id past the experts, whose output is written as 0).
template <int TD, int G, int NU, int NCW>
__global__ void __launch_bounds__(256)
    k_down_slots(const uint32_t *hprep, const uint32_t *slots, int n, const uint8_t *wd, int n_experts, int I, int H,
                 void *out, int odt) {
  constexpr int RB = 2, SPW = 64 / G;
  static_assert(NU == 1 || G == 64, "two units a lane only at one slot a wavefront");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int P = I / 64, CJ = RB * 9 * P / 4, CW = SPW * CJ;
  const int n0 = (blockIdx.x * 4 + wave) * RB;
  const int s0 = blockIdx.y * SPW, js = lane / G, p = lane % G;
  extern __shared__ u32x4 lds4[];
  u32x4 *st4 = lds4 + wave * CW;
  const uint32_t *stage = reinterpret_cast<const uint32_t *>(st4);

  const uint32_t id_l = slots[min(s0 + min(lane, SPW - 1), n - 1)];  // lane j < SPW: slot s0 + j's id
  const u32x4 *hb = reinterpret_cast<const u32x4 *>(hprep + size_t(min(s0 + js, n - 1)) * P * XS);
  u32x4 hq[NU][9];
#pragma unroll
  for (int a = 0; a < NU; ++a) {
    const int u = min(p + 64 * a, P - 1);
#pragma unroll
    for (int i = 0; i < 9; ++i) hq[a][i] = hb[u * 9 + i];
  }
  asm volatile("" ::: "memory");
  const size_t rowb = size_t(36) * P, nsafe = size_t(min(n0, H - RB));
  u32x4 w[NCW];
#pragma unroll
  for (int i = 0; i < NCW; ++i) {
    const int c = min(lane + 64 * i, CW - 1);
    const int j = c / CJ, cc = c - j * CJ;
    uint32_t e = uint32_t(__shfl(int(id_l), j, 64));
    e = e < uint32_t(n_experts) ? e : 0u;
    w[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(wd + (size_t(e) * H + nsafe) * rowb) + cc);
  }
  asm volatile("" ::: "memory");
  uint32_t xv[NU][32];
  float fa[NU], hs0[NU], hs1[NU];
  int uc[NU];
#pragma unroll
  for (int a = 0; a < NU; ++a) {
    const int u = p + 64 * a;
    uc[a] = min(u, P - 1);
    fa[a] = u < P ? 1.0f : 0.0f;
    unpack_unit(hq[a], xv[a]);
    h_unit_sums<TD>(xv[a], &hs0[a], &hs1[a]);
  }
#pragma unroll
  for (int i = 0; i < NCW; ++i) st4[min(lane + 64 * i, CW - 1)] = w[i];
  __builtin_amdgcn_wave_barrier();
  float acc[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) acc[r] = 0.0f;
#pragma unroll
  for (int a = 0; a < NU; ++a)
#pragma unroll
    for (int r = 0; r < RB; ++r)
      acc[r] = fmaf(fa[a], row_unit_dot_r<TD>(stage + (js * RB + r) * 9 * P, uc[a], xv[a], hs0[a], hs1[a]), acc[r]);
#pragma unroll
  for (int r = 0; r < RB; ++r) acc[r] = slot_sum<G>(acc[r]);
  const uint32_t e = uint32_t(__shfl(int(id_l), js, 64));
  if (p < RB && s0 + js < n)
    store_elt(out, size_t(s0 + js) * H + n0 + p, e < uint32_t(n_experts) ? (p == 0 ? acc[0] : acc[1]) : 0.0f, odt);
}

// Down of the same windows, unweighted: grid (H / 8, ceil(n / tr)), 256 threads; wavefront w of block (bx, y) takes
// output rows [(4 bx + w) 2, +2) for the prepared h rows [y tr, +tr), SPW rows of a run a pass on k_down_slots'
// lanes and arithmetic (the same staged rows, unit dots, weights and group sums). LDS: the window's h rows, its slot
// ids, each wavefront's 2 staged rows.
template <int TD, int G, int NU, int NCW>
__global__ void __launch_bounds__(256)
    k_down_runs_xr(const uint32_t *hprep, const uint32_t *slots, int n, int tr, const uint8_t *wd, int n_experts,
                   int I, int H, void *out, int odt) {
  constexpr int RB = 2, SPW = 64 / G;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int P = I / 64, CW = RB * 9 * P / 4;
  const int n0 = (blockIdx.x * 4 + wave) * RB;
  const int e0 = blockIdx.y * tr, ne = min(tr, n - e0);
  const int js = lane / G, p = lane % G;
  extern __shared__ u32x4 lds4[];
  u32x4 *hw = lds4;  // 9 P chunks a row
  uint32_t *sl = reinterpret_cast<uint32_t *>(lds4 + size_t(tr) * 9 * P);
  u32x4 *st4 = reinterpret_cast<u32x4 *>(sl + ((tr + 3) & ~3)) + wave * CW;
  const uint32_t *stage = reinterpret_cast<const uint32_t *>(st4);

  const size_t rowb = size_t(36) * P, nsafe = size_t(min(n0, H - RB));
  u32x4 w[NCW];
  auto fetch = [&](uint32_t e) {
    const u32x4 *src =
        reinterpret_cast<const u32x4 *>(wd + (size_t(e < uint32_t(n_experts) ? e : 0u) * H + nsafe) * rowb);
#pragma unroll
    for (int i = 0; i < NCW; ++i) w[i] = __builtin_nontemporal_load(src + min(lane + 64 * i, CW - 1));
  };
  fetch(slots[e0]);
  if (int(threadIdx.x) < ne) sl[threadIdx.x] = slots[e0 + threadIdx.x];
  {
    const u32x4 *src = reinterpret_cast<const u32x4 *>(hprep + size_t(e0) * P * XS);
    for (int c = threadIdx.x; c < ne * 9 * P; c += 256) hw[c] = src[c];
  }
  __syncthreads();
  if (n0 >= H) return;

  for (int r = 0; r < ne;) {
    const uint32_t e = sl[r];
    int r1 = r + 1;
    while (r1 < ne && sl[r1] == e) ++r1;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < NCW; ++i) st4[min(lane + 64 * i, CW - 1)] = w[i];
    if (r1 < ne) fetch(sl[r1]);
    __builtin_amdgcn_wave_barrier();
    const bool valid = e < uint32_t(n_experts);
    for (int q0 = r; q0 < r1; q0 += SPW) {
      const bool mine = q0 + js < r1;
      const size_t o = size_t(e0 + q0 + js) * H + n0 + p;
      if (!valid) {  // k_down_slots writes 0 for such an id
        if (p < RB && mine) store_elt(out, o, 0.0f, odt);
        continue;
      }
      const u32x4 *hb = hw + size_t(min(q0 + js, r1 - 1)) * 9 * P;
      float acc[RB];
#pragma unroll
      for (int rr = 0; rr < RB; ++rr) acc[rr] = 0.0f;
#pragma unroll
      for (int a = 0; a < NU; ++a) {
        const int u = p + 64 * a, uc = min(u, P - 1);
        const float fa = u < P ? 1.0f : 0.0f;
        uint32_t xv[32];
        unpack_unit(hb + uc * 9, xv);
        float x0, x1;
        h_unit_sums<TD>(xv, &x0, &x1);
#pragma unroll
        for (int rr = 0; rr < RB; ++rr)
          acc[rr] = fmaf(fa, row_unit_dot_r<TD>(stage + rr * 9 * P, uc, xv, x0, x1), acc[rr]);
      }
#pragma unroll
      for (int rr = 0; rr < RB; ++rr) acc[rr] = slot_sum<G>(acc[rr]);
      if (p < RB && mine) store_elt(out, o, p == 0 ? acc[0] : acc[1], odt);
    }
    r = r1;
  }
}

struct GateUpArgs {
  const uint32_t *xg_prep, *xu_prep;
  const void *x;
  int xdt;
  const uint32_t *slots;
  int n_slots, topk;
  const uint8_t *wg, *wu;
  int n_experts, H, I;
  float *h;
  uint32_t *hprep;
  int td;
  const float *logits;
  int ld_stride, norm;
  uint32_t *ids_out;
  float *scores_out;
  int ks = 0;  // slots a token when a shared expert is folded in (topk + 1); 0: topk
};

template <int TG, int TU, int RB, int NC, int NW>
static int launch_gate_up(const GateUpArgs &a, hipStream_t st) {
  const int P = a.H / 64;
  const size_t stage_dw = size_t(2) * RB * 9 * P;
  const size_t xraw_dw = a.xg_prep ? 0 : size_t(16) * P * (a.xdt == LMOE_F32 ? 4 : 2);
  const size_t lds = size_t(4) * ((TG == TU ? 1 : 2) * P * XS + std::max(NW * stage_dw, xraw_dw) +
                                  NW * 2 * RB * (P + 1));
  LMOE_REQUIRE(lds <= 160 * 1024, LMOE_ESHAPE, "lmoe_gemv_gate_up: hidden %d needs %zu bytes of LDS", a.H, lds);
  const dim3 grid((a.I + RB * NW - 1) / (RB * NW), a.n_slots);
  if (int rc = allow_lds(k_gate_up<TG, TU, RB, NC, NW>, lds, "lmoe_gemv_gate_up")) return rc;
  launch(k_gate_up<TG, TU, RB, NC, NW>, grid, dim3(64 * NW), lds, st, a.xg_prep, a.xu_prep, a.x,
                     a.xdt, a.slots, a.topk, a.wg, a.wu, a.n_experts, a.I, a.h, a.hprep, a.td, P, a.logits,
                     a.ld_stride, a.norm, a.ids_out, a.scores_out);
  LMOE_LAUNCHED("lmoe_gemv_gate_up");
  return 0;
}

// 2 rows a task when the row chunks split evenly (P even), else 4; NC covers a task's 16-byte chunks a lane.
// Where the fused top-k ranks: in each wavefront (the default: cfg2 in a HIP graph, 15.65 against 15.84 us a layer
// on one box), or with LMOE_GATE_UP_RANK=1 once a workgroup (rank256, one barrier before every weight load).
static bool gate_up_rank_wg() {
  static const bool wg = [] {
    const char *v = getenv("LMOE_GATE_UP_RANK");
    return v && v[0] == '1';
  }();
  return wg;
}

template <int TQ, int P, int RB, int NPL>
static int launch_gate_up_xr(const GateUpArgs &a, hipStream_t st) {
  const dim3 grid((a.I + 4 * RB - 1) / (4 * RB), a.n_slots);
  unsigned long long *tl = gate_up_rank_wg() ? nullptr : timeline_next(LMOE_TL_GATE_UP, int(grid.x * grid.y));
  auto kern = tl                 ? k_gate_up_xr<TQ, P, RB, NPL, false, false, true>
              : gate_up_rank_wg() ? k_gate_up_xr<TQ, P, RB, NPL, true>
                                  : k_gate_up_xr<TQ, P, RB, NPL, false>;
  launch(kern, grid, dim3(256), 0, st, a.xg_prep, a.slots, a.topk, a.wg, a.wu,
         a.n_experts, a.I, a.h, a.hprep, a.td, a.logits, a.ld_stride, a.norm, a.ids_out, a.scores_out,
         a.ks ? a.ks : a.topk, nullptr, 0, tl);
  LMOE_LAUNCHED("lmoe_gemv_gate_up");
  return 0;
}

// The drop-in chain's gate/up: raw x prepared in each workgroup, slots given (k_gate_up_xr's RAW form).
template <int TQ, int P>
static int launch_gate_up_xr_raw(const GateUpArgs &a, hipStream_t st) {
  constexpr int RB = 2;
  const dim3 grid((a.I + 4 * RB - 1) / (4 * RB), a.n_slots);
  launch(k_gate_up_xr<TQ, P, RB, 0, false, true>, grid, dim3(256), 0, st, nullptr, a.slots, a.topk, a.wg, a.wu,
         a.n_experts, a.I, a.h, a.hprep, a.td, nullptr, 0, 0, nullptr, nullptr, a.topk, a.x, a.xdt,
         static_cast<unsigned long long *>(nullptr));
  LMOE_LAUNCHED("lmoe_gemv_chain_gate_up");
  return 0;
}

template <int TQ, int P, int RB>
static int gate_up_xr_npl(const GateUpArgs &a, hipStream_t st) {
  if (!a.logits) return launch_gate_up_xr<TQ, P, RB, 0>(a, st);
  if (a.n_experts <= 64) return launch_gate_up_xr<TQ, P, RB, 1>(a, st);
  if (a.n_experts <= 128) return launch_gate_up_xr<TQ, P, RB, 2>(a, st);
  if (a.n_experts <= 256) return launch_gate_up_xr<TQ, P, RB, 4>(a, st);
  if (a.n_experts <= 512) return launch_gate_up_xr<TQ, P, RB, 8>(a, st);
  return launch_gate_up_xr<TQ, P, RB, 16>(a, st);
}

template <int TG, int TU>
static int gate_up_p(const GateUpArgs &a, hipStream_t st) {
  const int P = a.H / 64;
  // prepared activations, one block type, 32 or 64 units a row: the register-resident kernel
  if (TG == TU && a.xg_prep && a.I % 2 == 0) {
    if (P == 32) return gate_up_xr_npl<TG, 32, 2>(a, st);
    if (P == 64) return gate_up_xr_npl<TG, 64, 2>(a, st);
  }
  if (a.ks) return fail(LMOE_ESHAPE, "lmoe_moe_gate_up_ext: a folded shared expert takes H = 2048 or 4096 and one type");
  if (P % 2 == 0) {
    const int nc = (2 * 9 * P / 4 + 63) / 64;
    if (nc <= 2) return launch_gate_up<TG, TU, 2, 2, 4>(a, st);
    if (nc <= 3) return launch_gate_up<TG, TU, 2, 3, 4>(a, st);
    if (nc <= 5) return launch_gate_up<TG, TU, 2, 5, 4>(a, st);
    if (nc <= 6) return launch_gate_up<TG, TU, 2, 6, 4>(a, st);
  }
  const int nc = (9 * P + 63) / 64;
  if (nc <= 2) return launch_gate_up<TG, TU, 4, 2, 4>(a, st);
  if (nc <= 4) return launch_gate_up<TG, TU, 4, 4, 4>(a, st);
  if (nc <= 6) return launch_gate_up<TG, TU, 4, 6, 4>(a, st);
  if (nc <= 9) return launch_gate_up<TG, TU, 4, 9, 2>(a, st);
  if (nc <= 12) return launch_gate_up<TG, TU, 4, 12, 2>(a, st);
  return fail(LMOE_ESHAPE, "lmoe_gemv_gate_up: hidden %d is above the 5376 this kernel stages", a.H);
}

static int check_matrix(const char *fn, int type, int rows, int cols, const void *buf) {
  LMOE_REQUIRE(qtype_ok(type), LMOE_ETYPE, "%s: ggml type %d is not supported (Q4_0 = 2, Q4_K = 12)", fn, type);
  LMOE_REQUIRE(cols > 0 && cols % block_weights(type) == 0 && cols % 64 == 0, LMOE_ESHAPE,
               "%s: row length %d is not a multiple of %d", fn, cols, type == LMOE_Q4_K ? 256 : 64);
  LMOE_REQUIRE(rows > 0 && rows % 4 == 0, LMOE_ESHAPE, "%s: %d rows is not a multiple of 4", fn, rows);
  LMOE_REQUIRE(buf && aligned16(buf), LMOE_EALIGN, "%s: expert buffer must be 16-byte aligned", fn);
  return 0;
}

static int gate_up(const char *fn, const GateUpArgs &a_in, int type_g, int type_u, void *stream) {
  // a Q6_K down takes h prepared in the Q4_K order, a Q8_0 down in the Q4_0 order (their kernels pair the values as
  // those types' nibble words do)
  GateUpArgs a = a_in;
  if (a.hprep && a.td == LMOE_Q6_K) a.td = LMOE_Q4_K;
  if (a.hprep && a.td == LMOE_Q8_0) a.td = LMOE_Q4_0;
  LMOE_REQUIRE(a.n_slots >= 0 && a.topk > 0 && a.n_slots % (a.ks ? a.ks : a.topk) == 0, LMOE_ESHAPE,
               "%s: %d slots is not a multiple of topk %d", fn, a.n_slots, a.topk);
  LMOE_REQUIRE(a.n_experts > 0, LMOE_ESHAPE, "%s: no experts", fn);
  if (!qtype_ok(type_g) || !qtype_ok(type_u)) {  // a type beyond Q4_0 / Q4_K: the general chain
    LMOE_REQUIRE(qtype_any(type_g) && qtype_any(type_u), LMOE_ETYPE,
                 "%s: ggml types %d/%d are not supported (Q4_0 = 2, Q4_1 = 3, Q8_0 = 8, Q4_K = 12, Q5_K = 13, "
                 "Q6_K = 14)", fn, type_g, type_u);
    LMOE_REQUIRE((a.x || a.n_slots == 0) && !a.hprep && !a.logits && !a.xg_prep, LMOE_ETYPE,
                 "%s: ggml types %d/%d run on the general chain only (raw x in, float32 h out)", fn, type_g, type_u);
    return gate_up_any(fn, a.x, a.xdt, a.slots, a.n_slots, a.topk, a.wg, a.wu, type_g, type_u, a.n_experts, a.H,
                       a.I, a.h, (hipStream_t)stream);
  }
  if (int rc = check_matrix(fn, type_g, a.I, a.H, a.wg)) return rc;
  if (int rc = check_matrix(fn, type_u, a.I, a.H, a.wu)) return rc;
  LMOE_REQUIRE(!a.hprep || qtype_ok(a.td), LMOE_ETYPE, "%s: ggml type %d is not supported (Q4_0 = 2, Q4_K = 12)",
               fn, a.td);
  LMOE_REQUIRE(!a.hprep || (a.I % 64 == 0 && (a.td != LMOE_Q4_K || a.I % 256 == 0)), LMOE_ESHAPE,
               "%s: width %d cannot be prepared for ggml type %d", fn, a.I, a.td);
  if (a.n_slots == 0) return 0;
  LMOE_REQUIRE((a.slots || a.logits) && (a.h || a.hprep), LMOE_EINVAL, "%s: null pointer", fn);
  LMOE_REQUIRE(!a.logits || (a.ids_out && a.scores_out && a.topk <= 32 && a.topk <= a.n_experts &&
                                         a.n_experts <= 1024),
               LMOE_ESHAPE, "%s: top-k %d of %d experts is outside what the fused router takes", fn, a.topk,
               a.n_experts);
  hipStream_t st = (hipStream_t)stream;
  if (type_g == LMOE_Q4_0 && type_u == LMOE_Q4_0) return gate_up_p<LMOE_Q4_0, LMOE_Q4_0>(a, st);
  if (type_g == LMOE_Q4_K && type_u == LMOE_Q4_K) return gate_up_p<LMOE_Q4_K, LMOE_Q4_K>(a, st);
  if (type_g == LMOE_Q4_0) return gate_up_p<LMOE_Q4_0, LMOE_Q4_K>(a, st);
  return gate_up_p<LMOE_Q4_K, LMOE_Q4_0>(a, st);
}

struct DownArgs {
  const uint32_t *hprep;
  int has_sums;
  const float *h;
  const uint32_t *ids;
  const float *scores;
  int T, k;
  const uint8_t *wd;
  int type_d, n_experts, I, H;
  const float *shared, *gate;
  int gate_stride;
  const void *residual;
  int rdt;
  void *out;
  int odt;
};

static int down(const char *fn, const DownArgs &a, void *stream) {
  LMOE_REQUIRE(dtype_ok(a.odt) && (!a.residual || dtype_ok(a.rdt)), LMOE_EINVAL, "%s: bad dtype", fn);
  LMOE_REQUIRE(a.T >= 0 && a.k > 0 && a.k <= 32, LMOE_ESHAPE, "%s: k %d is outside 1..32", fn, a.k);
  LMOE_REQUIRE(a.n_experts > 0, LMOE_ESHAPE, "%s: no experts", fn);
  LMOE_REQUIRE(!a.shared == !a.gate, LMOE_EINVAL, "%s: shared and gate go together", fn);
  if (!qtype_ok(a.type_d)) {  // a type beyond Q4_0 / Q4_K: the general chain
    // Q6_K and Q8_0 also read h prepared in the Q4_K / Q4_0 order
    if (a.hprep && (a.type_d == LMOE_Q6_K || a.type_d == LMOE_Q8_0))
      return down_packed_prepped(fn, a.type_d, a.hprep, a.ids, a.scores, a.T, a.k, a.wd, a.n_experts, a.I, a.H,
                                 a.shared, a.gate, a.gate_stride, a.residual, a.rdt, a.out, a.odt,
                                 (hipStream_t)stream);
    LMOE_REQUIRE(!a.hprep, LMOE_ETYPE, "%s: ggml type %d runs on the general chain only (float32 h in)", fn,
                 a.type_d);
    LMOE_REQUIRE(a.T == 0 || aligned16(a.h), LMOE_EALIGN, "%s: h must be 16-byte aligned", fn);
    return down_any(fn, a.h, a.ids, a.scores, a.T, a.k, a.wd, a.type_d, a.n_experts, a.I, a.H, a.shared, a.gate,
                    a.gate_stride, a.residual, a.rdt, a.out, a.odt, (hipStream_t)stream);
  }
  if (int rc = check_matrix(fn, a.type_d, a.H, a.I, a.wd)) return rc;
  if (a.T == 0) return 0;
  LMOE_REQUIRE((a.h || a.hprep) && a.ids && a.out, LMOE_EINVAL, "%s: null pointer", fn);
  LMOE_REQUIRE(a.hprep ? aligned16(a.hprep) : aligned16(a.h), LMOE_EALIGN, "%s: h must be 16-byte aligned", fn);
  hipStream_t st = (hipStream_t)stream;
  {  // prepared h, at most 128 units a token, P even, H a multiple of 8: the register-resident kernel
    const int P = a.I / 64, U = a.k * P, CW = a.k * 9 * P / 2;
    const int kh = (a.k + 1) / 2, Uh = kh * P, CWh = kh * 9 * P / 2;
    // Two wavefronts a row pair, half of the experts each, wherever both halves fit (k >= 2): twice the workgroups
    // of one wavefront a row pair, so two wavefronts a SIMD have their loads in flight (cfg2 48-layer graph 14.72 ->
    // 14.39 us a layer, cfg5 24.15 -> 23.62; four wavefronts a row pair measured 15.21 and 25.5). Up to 256 units a
    // token it is the only register-resident form (cfg1 with its shared expert folded in: 8 experts of 22 units).
    // LMOE_DOWN_KS=1 keeps one wavefront a row pair where a token has at most 128 units.
    const char *ks_env = getenv("LMOE_DOWN_KS");
    const bool ks1 = ks_env && atoi(ks_env) == 1 && U <= 128 && CW <= 64 * 9;
    if (a.hprep && a.k >= 2 && !ks1 && Uh <= 128 && P % 2 == 0 && a.H % 4 == 0 && CWh <= 64 * 9) {
      const int NU = Uh <= 64 ? 1 : 2, ncw = (CWh + 63) / 64, hl = (8 * Uh + 63) / 64;
      // the h chunks as one run through LDS where that saves loads: 6 a lane at 48 units (cfg2, cfg5), 11 at 88
      // (cfg1), against 8 NU
      const int HLr = getenv("LMOE_DOWN_HL") && atoi(getenv("LMOE_DOWN_HL")) == 0 ? 0 : hl;
      // eight wavefronts a workgroup (four row pairs) where H allows: the four over the same experts share one copy
      // of their h half, half the h reads of four (LMOE_DOWN_WG8=0 keeps four)
      const bool wg8 = a.H % 8 == 0 && !(getenv("LMOE_DOWN_WG8") && atoi(getenv("LMOE_DOWN_WG8")) == 0);
      const int nwg = wg8 ? 8 : 4;
      unsigned long long *tl = timeline_next(LMOE_TL_DOWN, (a.H / nwg) * a.T);
      auto go = [&](auto td, auto nu, auto nc) {
        constexpr int TD = decltype(td)::value, N = decltype(nu)::value, C = decltype(nc)::value;
        auto run = [&](auto hlc) {
          constexpr int HLc = decltype(hlc)::value;
          const size_t lds = size_t(16) * (size_t(nwg) * CWh + (HLc > 0 ? 2 : nwg) * 64 * HLc);
          if (wg8)
            launch(tl ? k_down_xr<TD, N, C, 2, HLc, true, 8> : k_down_xr<TD, N, C, 2, HLc, false, 8>,
                   dim3(a.H / 8, a.T), dim3(512), lds, st, a.hprep, a.ids, a.scores, a.k, a.wd, a.n_experts, a.I,
                   a.H, a.shared, a.gate, a.gate_stride, a.residual, a.rdt, a.out, a.odt, tl);
          else
            launch(tl ? k_down_xr<TD, N, C, 2, HLc, true> : k_down_xr<TD, N, C, 2, HLc>, dim3(a.H / 4, a.T),
                   dim3(256), lds, st, a.hprep, a.ids, a.scores, a.k, a.wd, a.n_experts, a.I, a.H, a.shared, a.gate,
                   a.gate_stride, a.residual, a.rdt, a.out, a.odt, tl);
        };
        if (N == 1 && HLr == 6)
          run(std::integral_constant<int, 6>());
        else if (N == 2 && HLr == 11)
          run(std::integral_constant<int, 11>());
        else
          run(std::integral_constant<int, 0>());
      };
      using I1 = std::integral_constant<int, 1>;
      using I2 = std::integral_constant<int, 2>;
      using C4 = std::integral_constant<int, 4>;
      using C5 = std::integral_constant<int, 5>;
      using C7 = std::integral_constant<int, 7>;
      using C9 = std::integral_constant<int, 9>;
      auto by_c = [&](auto td, auto nu) {
        if (ncw <= 4) go(td, nu, C4());
        else if (ncw <= 5) go(td, nu, C5());
        else if (ncw <= 7) go(td, nu, C7());
        else go(td, nu, C9());
      };
      auto by_nu = [&](auto td) {
        if (NU == 1) by_c(td, I1());
        else by_c(td, I2());
      };
      if (a.type_d == LMOE_Q4_0)
        by_nu(std::integral_constant<int, LMOE_Q4_0>());
      else
        by_nu(std::integral_constant<int, LMOE_Q4_K>());
      LMOE_LAUNCHED(fn);
      return 0;
    }
    if (a.hprep && U <= 128 && P % 2 == 0 && a.H % 8 == 0 && CW <= 64 * 9) {
      const int NU = U <= 64 ? 1 : 2, ncw = (CW + 63) / 64;
      auto go = [&](auto td, auto nu, auto nc) {
        constexpr int TD = decltype(td)::value, N = decltype(nu)::value, C = decltype(nc)::value;
        launch(k_down_xr<TD, N, C>, dim3(a.H / 8, a.T), dim3(256), size_t(4) * 4 * CW * 4, st, a.hprep, a.ids,
               a.scores, a.k, a.wd, a.n_experts, a.I, a.H, a.shared, a.gate, a.gate_stride, a.residual, a.rdt, a.out,
               a.odt, static_cast<unsigned long long *>(nullptr));
      };
      using I1 = std::integral_constant<int, 1>;
      using I2 = std::integral_constant<int, 2>;
      using C5 = std::integral_constant<int, 5>;
      using C7 = std::integral_constant<int, 7>;
      using C9 = std::integral_constant<int, 9>;
      auto by_c = [&](auto td, auto nu) {
        if (ncw <= 5) go(td, nu, C5());
        else if (ncw <= 7) go(td, nu, C7());
        else go(td, nu, C9());
      };
      auto by_nu = [&](auto td) {
        if (NU == 1) by_c(td, I1());
        else by_c(td, I2());
      };
      if (a.type_d == LMOE_Q4_0)
        by_nu(std::integral_constant<int, LMOE_Q4_0>());
      else
        by_nu(std::integral_constant<int, LMOE_Q4_K>());
      LMOE_LAUNCHED(fn);
      return 0;
    }
  }
  constexpr int NW = 2, NC = 16;
  const int P = a.I / 64;
  const int RB = P % 2 == 0 ? 2 : 4;
  const size_t stage_dw = size_t(a.k) * RB * 9 * P;
  const size_t hraw_dw = a.hprep ? 0 : size_t(a.k) * a.I;
  const size_t lds = size_t(4) * (size_t(a.k) * P * XS + 64 + std::max(NW * stage_dw, hraw_dw) +
                                  NW * RB * (a.k * P + 1));
  LMOE_REQUIRE(lds <= 160 * 1024, LMOE_ESHAPE, "%s: k %d at width %d needs %zu bytes of LDS", fn, a.k, a.I, lds);
  const dim3 grid((a.H + RB * NW - 1) / (RB * NW), a.T);
  // weights fetched into registers ahead of the h staging when a wavefront's k RB rows fit in NC chunks a lane
  const bool pre = size_t(a.k) * RB * 9 * P / 4 <= size_t(64) * NC;
  auto pick = [&](auto td, auto rb) {
    constexpr int TD = decltype(td)::value, R = decltype(rb)::value;
    if (a.hprep) return pre ? k_down_combine<TD, R, NC, NW, true, true> : k_down_combine<TD, R, NC, NW, true, false>;
    return pre ? k_down_combine<TD, R, NC, NW, false, true> : k_down_combine<TD, R, NC, NW, false, false>;
  };
  using Q0 = std::integral_constant<int, LMOE_Q4_0>;
  using QK = std::integral_constant<int, LMOE_Q4_K>;
  using R2 = std::integral_constant<int, 2>;
  using R4 = std::integral_constant<int, 4>;
  auto kern = a.type_d == LMOE_Q4_0 ? (RB == 2 ? pick(Q0(), R2()) : pick(Q0(), R4()))
                                    : (RB == 2 ? pick(QK(), R2()) : pick(QK(), R4()));
  if (int rc = allow_lds(kern, lds, fn)) return rc;
  launch(kern, grid, dim3(64 * NW), lds, st, a.hprep, a.has_sums, a.h, a.ids, a.scores, a.k, a.wd,
                     a.n_experts, a.I, a.H, a.shared, a.gate, a.gate_stride, a.residual, a.rdt, a.out, a.odt);
  LMOE_LAUNCHED(fn);
  return 0;
}

// Rows a window of the run kernels: `want` (1..64), lowered until the window's LDS fits `cap` bytes.
static int runs_window(int want, size_t fixed, size_t per_row, size_t cap) {
  int tr = std::min(std::max(want, 1), 64);
  while (tr > 1 && fixed + per_row * tr > cap) --tr;
  return tr;
}

// 16-byte chunks a lane a matrix the run kernels hold for c chunks a wavefront: a compiled count at or above it
static int runs_nc(int c) {
  const int nc = (c + 63) / 64;
  return nc <= 1 ? 1 : nc <= 2 ? 2 : nc <= 3 ? 3 : nc <= 5 ? 5 : nc <= 6 ? 6 : nc <= 9 ? 9 : 0;
}

template <int TG, int TU, int RB, int NW>
static int launch_gate_up_runs(int nc, dim3 grid, size_t lds, hipStream_t st, const void *x, int xdt,
                               const uint32_t *slots, int n, int tr, const uint8_t *wg, const uint8_t *wu,
                               int n_experts, int I, int P, float *h) {
  const char *fn = "lmoe_gemv_gate_up_runs";
  auto go = [&](auto kern) {
    if (int rc = allow_lds(kern, lds, fn)) return rc;
    launch(kern, grid, dim3(64 * NW), lds, st, x, xdt, slots, n, tr, wg, wu, n_experts, I, P, h);
    LMOE_LAUNCHED(fn);
    return 0;
  };
  switch (nc) {
    case 1: return go(k_gate_up_runs<TG, TU, RB, NW, 1>);
    case 2: return go(k_gate_up_runs<TG, TU, RB, NW, 2>);
    case 3: return go(k_gate_up_runs<TG, TU, RB, NW, 3>);
    case 5: return go(k_gate_up_runs<TG, TU, RB, NW, 5>);
    case 6: return go(k_gate_up_runs<TG, TU, RB, NW, 6>);
    default: return go(k_gate_up_runs<TG, TU, RB, NW, 9>);
  }
}

static int gate_up_runs(const void *x, int xdt, const uint32_t *slots, int n, int tr_want, const uint8_t *wg,
                        const uint8_t *wu, int tg, int tu, int n_experts, int H, int I, float *h, hipStream_t st) {
  const char *fn = "lmoe_gemv_gate_up_runs";
  LMOE_REQUIRE(dtype_ok(xdt), LMOE_EINVAL, "%s: x dtype %d is not F32, F16 or BF16", fn, xdt);
  LMOE_REQUIRE(qtype_ok(tg) && qtype_ok(tu), LMOE_ETYPE, "%s: the run kernels take Q4_0 / Q4_K (got %d/%d)", fn, tg,
               tu);
  LMOE_REQUIRE(n_experts > 0 && n >= 0 && tr_want >= 1, LMOE_ESHAPE, "%s: %d experts, %d rows, window %d", fn,
               n_experts, n, tr_want);
  if (int rc = check_matrix(fn, tg, I, H, wg)) return rc;
  if (int rc = check_matrix(fn, tu, I, H, wu)) return rc;
  constexpr int NW = 4;
  const int P = H / 64, RB = P % 2 == 0 ? 2 : 4;
  const int nc = runs_nc(RB * 9 * P / 4);
  LMOE_REQUIRE(nc > 0, LMOE_ESHAPE, "%s: hidden %d needs more weight chunks a lane than the run kernels hold", fn, H);
  if (n == 0) return 0;
  LMOE_REQUIRE(x && slots && h && aligned16(x), LMOE_EALIGN, "%s: null or unaligned pointer", fn);
  const size_t prow = size_t(P) * XS * (tg == tu ? 1 : 2), stage = size_t(NW) * 2 * RB * 9 * P;
  const size_t red = size_t(NW) * kRunQ * 2 * RB * (P + 1);
  const int tr = runs_window(tr_want, 4 * (stage + red + 64), 4 * prow, 80 * 1024);
  const size_t lds = 4 * (tr * prow + ((tr + 3) & ~3) + stage + red);
  LMOE_REQUIRE(lds <= 160 * 1024, LMOE_ESHAPE, "%s: hidden %d needs %zu bytes of LDS", fn, H, lds);
  const dim3 grid((I + RB * NW - 1) / (RB * NW), (n + tr - 1) / tr);
  constexpr int Q0 = LMOE_Q4_0, QK = LMOE_Q4_K;
  auto go = [&](auto g, auto u, auto rb) {
    constexpr int G = decltype(g)::value, UU = decltype(u)::value, R = decltype(rb)::value;
    return launch_gate_up_runs<G, UU, R, NW>(nc, grid, lds, st, x, xdt, slots, n, tr, wg, wu, n_experts, I, P, h);
  };
  using T0 = std::integral_constant<int, Q0>;
  using TK = std::integral_constant<int, QK>;
  using R2 = std::integral_constant<int, 2>;
  using R4 = std::integral_constant<int, 4>;
  if (RB == 2) {
    if (tg == Q0) return tu == Q0 ? go(T0(), T0(), R2()) : go(T0(), TK(), R2());
    return tu == Q0 ? go(TK(), T0(), R2()) : go(TK(), TK(), R2());
  }
  if (tg == Q0) return tu == Q0 ? go(T0(), T0(), R4()) : go(T0(), TK(), R4());
  return tu == Q0 ? go(TK(), T0(), R4()) : go(TK(), TK(), R4());
}

static int down_runs(const float *h, const uint32_t *slots, int n, int tr_want, const uint8_t *wd, int td,
                     int n_experts, int I, int H, void *out, int odt, hipStream_t st) {
  const char *fn = "lmoe_gemv_down_runs";
  LMOE_REQUIRE(dtype_ok(odt), LMOE_EINVAL, "%s: bad dtype", fn);
  LMOE_REQUIRE(qtype_ok(td), LMOE_ETYPE, "%s: the run kernels take Q4_0 / Q4_K (got %d)", fn, td);
  LMOE_REQUIRE(n_experts > 0 && n >= 0 && tr_want >= 1, LMOE_ESHAPE, "%s: %d experts, %d rows, window %d", fn,
               n_experts, n, tr_want);
  if (int rc = check_matrix(fn, td, H, I, wd)) return rc;
  constexpr int NW = 4;
  const int P = I / 64, RB = P % 2 == 0 ? 2 : 4;
  const int nc = runs_nc(RB * 9 * P / 4);
  LMOE_REQUIRE(nc > 0, LMOE_ESHAPE, "%s: width %d needs more weight chunks a lane than the run kernels hold", fn, I);
  if (n == 0) return 0;
  LMOE_REQUIRE(h && slots && out && aligned16(h), LMOE_EALIGN, "%s: null or unaligned pointer", fn);
  const size_t prow = size_t(P) * XS, stage = size_t(NW) * RB * 9 * P, red = size_t(NW) * kRunQ * RB * (P + 1);
  const int tr = runs_window(tr_want, 4 * (stage + red + 64), 4 * prow, 80 * 1024);
  const size_t lds = 4 * (tr * prow + ((tr + 3) & ~3) + stage + red);
  LMOE_REQUIRE(lds <= 160 * 1024, LMOE_ESHAPE, "%s: width %d needs %zu bytes of LDS", fn, I, lds);
  const dim3 grid((H + RB * NW - 1) / (RB * NW), (n + tr - 1) / tr);
  auto go = [&](auto kern) {
    if (int rc = allow_lds(kern, lds, fn)) return rc;
    launch(kern, grid, dim3(64 * NW), lds, st, h, slots, n, tr, wd, n_experts, I, H, out, odt);
    LMOE_LAUNCHED(fn);
    return 0;
  };
  auto by_nc = [&](auto td_, auto rb) {
    constexpr int D = decltype(td_)::value, R = decltype(rb)::value;
    switch (nc) {
      case 1: return go(k_down_runs<D, R, NW, 1>);
      case 2: return go(k_down_runs<D, R, NW, 2>);
      case 3: return go(k_down_runs<D, R, NW, 3>);
      case 5: return go(k_down_runs<D, R, NW, 5>);
      case 6: return go(k_down_runs<D, R, NW, 6>);
      default: return go(k_down_runs<D, R, NW, 9>);
    }
  };
  using T0 = std::integral_constant<int, LMOE_Q4_0>;
  using TK = std::integral_constant<int, LMOE_Q4_K>;
  using R2 = std::integral_constant<int, 2>;
  using R4 = std::integral_constant<int, 4>;
  if (td == LMOE_Q4_0) return RB == 2 ? by_nc(T0(), R2()) : by_nc(T0(), R4());
  return RB == 2 ? by_nc(TK(), R2()) : by_nc(TK(), R4());
}

static int gate_up_runs_prepped(const uint32_t *xprep, const uint32_t *slots, int n, int tr_want, const uint8_t *wg,
                                const uint8_t *wu, int type, int n_experts, int H, int I, float *h, uint32_t *hprep,
                                int td, hipStream_t st) {
  const char *fn = "lmoe_gemv_gate_up_runs_prepped";
  LMOE_REQUIRE(qtype_ok(type), LMOE_ETYPE, "%s: the run kernels take Q4_0 / Q4_K (got %d)", fn, type);
  LMOE_REQUIRE(n_experts > 0 && n >= 0 && tr_want >= 1, LMOE_ESHAPE, "%s: %d experts, %d rows, window %d", fn,
               n_experts, n, tr_want);
  LMOE_REQUIRE((H == 2048 || H == 4096) && I % 2 == 0, LMOE_ESHAPE,
               "%s: takes the register-resident form, hidden 2048 or 4096 and an even width (got %d, %d)", fn, H, I);
  if (int rc = check_matrix(fn, type, I, H, wg)) return rc;
  if (int rc = check_matrix(fn, type, I, H, wu)) return rc;
  if (hprep && td == LMOE_Q6_K) td = LMOE_Q4_K;  // the orders lmoe_gemv_gate_up_prepped writes for these downs
  if (hprep && td == LMOE_Q8_0) td = LMOE_Q4_0;
  LMOE_REQUIRE(!hprep || (qtype_ok(td) && I % 64 == 0 && (td != LMOE_Q4_K || I % 256 == 0)), LMOE_ESHAPE,
               "%s: width %d cannot be prepared for ggml type %d", fn, I, td);
  LMOE_REQUIRE(h || hprep, LMOE_EINVAL, "%s: neither h nor its prepared rows asked for", fn);
  if (n == 0) return 0;
  LMOE_REQUIRE(xprep && slots && aligned16(xprep), LMOE_EALIGN, "%s: null or unaligned pointer", fn);
  const int P = H / 64;
  const size_t prow = size_t(P) * XS, stage = size_t(4) * 2 * 2 * 9 * P;
  const int tr = runs_window(tr_want, 4 * (stage + 64), 4 * prow, 80 * 1024);
  const size_t lds = 4 * (tr * prow + ((tr + 3) & ~3) + stage);
  const dim3 grid((I + 7) / 8, (n + tr - 1) / tr);
  auto go = [&](auto kern) {
    if (int rc = allow_lds(kern, lds, fn)) return rc;
    launch(kern, grid, dim3(256), lds, st, xprep, slots, n, tr, wg, wu, n_experts, I, h, hprep, td);
    LMOE_LAUNCHED(fn);
    return 0;
  };
  if (type == LMOE_Q4_0) return P == 32 ? go(k_gate_up_runs_xr<LMOE_Q4_0, 32>) : go(k_gate_up_runs_xr<LMOE_Q4_0, 64>);
  return P == 32 ? go(k_gate_up_runs_xr<LMOE_Q4_K, 32>) : go(k_gate_up_runs_xr<LMOE_Q4_K, 64>);
}

// Lanes a slot's units take in k_down_slots / k_down_runs_xr (a power of two, 16 at least, 64 at most) and units a
// lane (2 past 64 units)
static int slot_group(int P) { return P <= 16 ? 16 : P <= 32 ? 32 : 64; }

static int check_down_slots(const char *fn, int td, int n_experts, int I, int H, const uint8_t *wd, int odt) {
  LMOE_REQUIRE(dtype_ok(odt), LMOE_EINVAL, "%s: bad dtype", fn);
  LMOE_REQUIRE(qtype_ok(td), LMOE_ETYPE, "%s: takes Q4_0 / Q4_K (got %d)", fn, td);
  LMOE_REQUIRE(n_experts > 0, LMOE_ESHAPE, "%s: no experts", fn);
  if (int rc = check_matrix(fn, td, H, I, wd)) return rc;
  const int P = I / 64;
  LMOE_REQUIRE(P % 2 == 0 && P <= 128 && H % 8 == 0, LMOE_ESHAPE,
               "%s: takes a width that is a multiple of 128 up to 8192 and a hidden size that is a multiple of 8 "
               "(got %d, %d)", fn, I, H);
  return 0;
}

static int down_slots(const uint32_t *hprep, const uint32_t *slots, int n, const uint8_t *wd, int td, int n_experts,
                      int I, int H, void *out, int odt, hipStream_t st) {
  const char *fn = "lmoe_gemv_chain_down";
  if (int rc = check_down_slots(fn, td, n_experts, I, H, wd, odt)) return rc;
  if (n == 0) return 0;
  LMOE_REQUIRE(hprep && slots && out && aligned16(hprep), LMOE_EALIGN, "%s: null or unaligned pointer", fn);
  const int P = I / 64, G = slot_group(P), spw = 64 / G, cw = spw * 9 * P / 2, ncw = (cw + 63) / 64;
  const size_t lds = size_t(16) * 4 * cw;
  const dim3 grid(H / 8, (n + spw - 1) / spw);
  auto go = [&](auto kern) {
    if (int rc = allow_lds(kern, lds, fn)) return rc;
    launch(kern, grid, dim3(256), lds, st, hprep, slots, n, wd, n_experts, I, H, out, odt);
    LMOE_LAUNCHED(fn);
    return 0;
  };
  auto by_nc = [&](auto td_, auto g_, auto nu_) {
    constexpr int D = decltype(td_)::value, GG = decltype(g_)::value, N = decltype(nu_)::value;
    if (ncw <= 2) return go(k_down_slots<D, GG, N, 2>);
    if (ncw <= 3) return go(k_down_slots<D, GG, N, 3>);
    if (ncw <= 4) return go(k_down_slots<D, GG, N, 4>);
    if (ncw <= 5) return go(k_down_slots<D, GG, N, 5>);
    return go(k_down_slots<D, GG, N, 9>);
  };
  auto by_g = [&](auto td_) {
    if (G == 16) return by_nc(td_, std::integral_constant<int, 16>(), std::integral_constant<int, 1>());
    if (G == 32) return by_nc(td_, std::integral_constant<int, 32>(), std::integral_constant<int, 1>());
    if (P <= 64) return by_nc(td_, std::integral_constant<int, 64>(), std::integral_constant<int, 1>());
    return by_nc(td_, std::integral_constant<int, 64>(), std::integral_constant<int, 2>());
  };
  return td == LMOE_Q4_0 ? by_g(std::integral_constant<int, LMOE_Q4_0>())
                         : by_g(std::integral_constant<int, LMOE_Q4_K>());
}

static int down_runs_prepped(const uint32_t *hprep, const uint32_t *slots, int n, int tr_want, const uint8_t *wd,
                             int td, int n_experts, int I, int H, void *out, int odt, hipStream_t st) {
  const char *fn = "lmoe_gemv_down_runs_prepped";
  LMOE_REQUIRE(tr_want >= 1 && n >= 0, LMOE_ESHAPE, "%s: %d rows, window %d", fn, n, tr_want);
  if (int rc = check_down_slots(fn, td, n_experts, I, H, wd, odt)) return rc;
  if (n == 0) return 0;
  LMOE_REQUIRE(hprep && slots && out && aligned16(hprep), LMOE_EALIGN, "%s: null or unaligned pointer", fn);
  const int P = I / 64, G = slot_group(P), cw = 9 * P / 2, ncw = (cw + 63) / 64;
  const size_t prow = size_t(P) * XS, stage = size_t(4) * 4 * cw;
  const int tr = runs_window(tr_want, 4 * (stage + 64), 4 * prow, 80 * 1024);
  const size_t lds = 4 * (tr * prow + ((tr + 3) & ~3) + stage);
  const dim3 grid(H / 8, (n + tr - 1) / tr);
  auto go = [&](auto kern) {
    if (int rc = allow_lds(kern, lds, fn)) return rc;
    launch(kern, grid, dim3(256), lds, st, hprep, slots, n, tr, wd, n_experts, I, H, out, odt);
    LMOE_LAUNCHED(fn);
    return 0;
  };
  auto by_nc = [&](auto td_, auto g_, auto nu_) {
    constexpr int D = decltype(td_)::value, GG = decltype(g_)::value, N = decltype(nu_)::value;
    if (ncw <= 1) return go(k_down_runs_xr<D, GG, N, 1>);
    if (ncw <= 2) return go(k_down_runs_xr<D, GG, N, 2>);
    if (ncw <= 3) return go(k_down_runs_xr<D, GG, N, 3>);
    if (ncw <= 5) return go(k_down_runs_xr<D, GG, N, 5>);
    return go(k_down_runs_xr<D, GG, N, 9>);
  };
  auto by_g = [&](auto td_) {
    if (G == 16) return by_nc(td_, std::integral_constant<int, 16>(), std::integral_constant<int, 1>());
    if (G == 32) return by_nc(td_, std::integral_constant<int, 32>(), std::integral_constant<int, 1>());
    if (P <= 64) return by_nc(td_, std::integral_constant<int, 64>(), std::integral_constant<int, 1>());
    return by_nc(td_, std::integral_constant<int, 64>(), std::integral_constant<int, 2>());
  };
  return td == LMOE_Q4_0 ? by_g(std::integral_constant<int, LMOE_Q4_0>())
                         : by_g(std::integral_constant<int, LMOE_Q4_K>());
}

static int chain_gate_up(const void *x, int xdt, const uint32_t *slots, int n, int topk, const uint8_t *wg,
                         const uint8_t *wu, int type, int n_experts, int H, int I, float *h, uint32_t *hprep, int td,
                         hipStream_t st) {
  const char *fn = "lmoe_gemv_chain_gate_up";
  LMOE_REQUIRE(dtype_ok(xdt), LMOE_EINVAL, "%s: x dtype %d is not F32, F16 or BF16", fn, xdt);
  LMOE_REQUIRE(qtype_ok(type), LMOE_ETYPE, "%s: takes Q4_0 / Q4_K (got %d)", fn, type);
  LMOE_REQUIRE(n_experts > 0 && n >= 0 && topk > 0 && n % topk == 0, LMOE_ESHAPE,
               "%s: %d experts, %d slots, topk %d", fn, n_experts, n, topk);
  LMOE_REQUIRE((H == 2048 || H == 4096) && I % 2 == 0, LMOE_ESHAPE,
               "%s: takes hidden 2048 or 4096 and an even width (got %d, %d)", fn, H, I);
  if (int rc = check_matrix(fn, type, I, H, wg)) return rc;
  if (int rc = check_matrix(fn, type, I, H, wu)) return rc;
  LMOE_REQUIRE(!hprep || (qtype_ok(td) && I % 64 == 0 && (td != LMOE_Q4_K || I % 256 == 0)), LMOE_ESHAPE,
               "%s: width %d cannot be prepared for ggml type %d", fn, I, td);
  LMOE_REQUIRE(h || hprep, LMOE_EINVAL, "%s: neither h nor its prepared rows asked for", fn);
  if (n == 0) return 0;
  LMOE_REQUIRE(x && slots && aligned16(x), LMOE_EALIGN, "%s: null or unaligned pointer", fn);
  GateUpArgs a{nullptr, nullptr, x, xdt, slots, n, topk, wg, wu, n_experts, H, I, h, hprep, td, nullptr, 0, 0,
               nullptr, nullptr};
  if (type == LMOE_Q4_0) return H == 2048 ? launch_gate_up_xr_raw<LMOE_Q4_0, 32>(a, st)
                                          : launch_gate_up_xr_raw<LMOE_Q4_0, 64>(a, st);
  return H == 2048 ? launch_gate_up_xr_raw<LMOE_Q4_K, 32>(a, st) : launch_gate_up_xr_raw<LMOE_Q4_K, 64>(a, st);
}

}  // namespace lmoe

using namespace lmoe;

extern "C" int lmoe_gemv_gate_up(const void *x, int xdtype, const uint32_t *slots, int n_slots, int topk,
                                 const uint8_t *wg, const uint8_t *wu, int type_g, int type_u, int n_experts, int H,
                                 int I, float *h, void *stream) {
  const char *fn = "lmoe_gemv_gate_up";
  LMOE_REQUIRE(dtype_ok(xdtype), LMOE_EINVAL, "%s: x dtype %d is not F32, F16 or BF16", fn, xdtype);
  LMOE_REQUIRE(n_slots == 0 || (x && aligned16(x)), LMOE_EALIGN, "%s: x must be 16-byte aligned", fn);
  GateUpArgs a{nullptr, nullptr, x, xdtype, slots, n_slots, topk, wg, wu, n_experts, H, I, h, nullptr, 0,
               nullptr, 0, 0, nullptr, nullptr};
  return gate_up(fn, a, type_g, type_u, stream);
}

extern "C" int lmoe_gemv_gate_up_prepped(const uint32_t *xg_prep, const uint32_t *xu_prep, const uint32_t *slots,
                                         int n_slots, int topk, const uint8_t *wg, const uint8_t *wu, int type_g,
                                         int type_u, int n_experts, int H, int I, float *h, uint32_t *hprep,
                                         int type_d, void *stream) {
  const char *fn = "lmoe_gemv_gate_up_prepped";
  LMOE_REQUIRE(n_slots == 0 || (xg_prep && aligned16(xg_prep) && (type_g == type_u || (xu_prep && aligned16(xu_prep)))),
               LMOE_EALIGN, "%s: prepared rows must be given and 16-byte aligned", fn);
  GateUpArgs a{xg_prep, type_g == type_u ? xg_prep : xu_prep, nullptr, 0, slots, n_slots, topk, wg, wu, n_experts,
               H, I, h, hprep, type_d, nullptr, 0, 0, nullptr, nullptr};
  return gate_up(fn, a, type_g, type_u, stream);
}

extern "C" int lmoe_moe_gate_up(const float *logits, int ld_stride, int T, int k, int norm, const uint32_t *xg_prep,
                                const uint32_t *xu_prep, const uint8_t *wg, const uint8_t *wu, int type_g,
                                int type_u, int n_experts, int H, int I, uint32_t *ids, float *scores,
                                uint32_t *hprep, int type_d, void *stream) {
  const char *fn = "lmoe_moe_gate_up";
  LMOE_REQUIRE(T == 0 || (logits && xg_prep && aligned16(xg_prep) && (type_g == type_u || (xu_prep && aligned16(xu_prep)))),
               LMOE_EALIGN, "%s: logits and 16-byte aligned prepared rows must be given", fn);
  LMOE_REQUIRE(ld_stride >= n_experts, LMOE_ESHAPE, "%s: logits row stride %d is below %d experts", fn, ld_stride,
               n_experts);
  GateUpArgs a{xg_prep, type_g == type_u ? xg_prep : xu_prep, nullptr, 0, nullptr, T * k, k, wg, wu, n_experts,
               H, I, nullptr, hprep, type_d, logits, ld_stride, norm, ids, scores};
  return gate_up(fn, a, type_g, type_u, stream);
}

extern "C" int lmoe_moe_gate_up_ext(const float *logits, int ld_stride, int T, int k, int norm,
                                    const uint32_t *xg_prep, const uint32_t *xu_prep, const uint8_t *wg,
                                    const uint8_t *wu, int type_g, int type_u, int n_experts, int H, int I,
                                    uint32_t *ids, float *scores, uint32_t *hprep, int type_d, int with_shared,
                                    void *stream) {
  const char *fn = "lmoe_moe_gate_up_ext";
  LMOE_REQUIRE(with_shared >= 0, LMOE_EINVAL, "%s: %d shared slices", fn, with_shared);
  if (!with_shared)
    return lmoe_moe_gate_up(logits, ld_stride, T, k, norm, xg_prep, xu_prep, wg, wu, type_g, type_u, n_experts, H,
                            I, ids, scores, hprep, type_d, stream);
  LMOE_REQUIRE(T == 0 || (logits && xg_prep && aligned16(xg_prep)), LMOE_EALIGN,
               "%s: logits and 16-byte aligned prepared rows must be given", fn);
  LMOE_REQUIRE(type_g == type_u, LMOE_ETYPE, "%s: a folded shared expert takes one type for gate and up", fn);
  LMOE_REQUIRE(ld_stride >= n_experts + 1, LMOE_ESHAPE,
               "%s: logits rows need the shared expert's gate logit at column %d (stride %d)", fn, n_experts,
               ld_stride);
  const int ks = k + with_shared;
  LMOE_REQUIRE(k >= 1 && ks <= 64, LMOE_ESHAPE, "%s: k %d with %d shared slices", fn, k, with_shared);
  GateUpArgs a{xg_prep, xg_prep, nullptr, 0, nullptr, T * ks, k, wg, wu, n_experts, H, I, nullptr, hprep,
               type_d, logits, ld_stride, norm, ids, scores, ks};
  return gate_up(fn, a, type_g, type_u, stream);
}

extern "C" int lmoe_moe_gate_up_h(const float *logits, int ld_stride, int T, int k, int norm, const uint32_t *x_prep,
                                  const uint8_t *wg, const uint8_t *wu, int type, int n_experts, int H, int I,
                                  uint32_t *ids, float *scores, float *h, int with_shared, void *stream) {
  const char *fn = "lmoe_moe_gate_up_h";
  LMOE_REQUIRE(with_shared >= 0, LMOE_EINVAL, "%s: %d shared slices", fn, with_shared);
  LMOE_REQUIRE(T == 0 || (logits && x_prep && aligned16(x_prep) && h), LMOE_EALIGN,
               "%s: logits, 16-byte aligned prepared rows and h must be given", fn);
  LMOE_REQUIRE((H == 2048 || H == 4096) && I % 2 == 0, LMOE_ESHAPE,
               "%s: takes the register-resident form, hidden 2048 or 4096 and an even width (got %d, %d)", fn, H, I);
  LMOE_REQUIRE(ld_stride >= n_experts + (with_shared ? 1 : 0), LMOE_ESHAPE,
               "%s: logits row stride %d is below %d experts%s", fn, ld_stride, n_experts,
               with_shared ? " and the shared gate logit" : "");
  const int ks = k + with_shared;
  LMOE_REQUIRE(k >= 1 && ks <= 64, LMOE_ESHAPE, "%s: k %d with %d shared slices", fn, k, with_shared);
  GateUpArgs a{x_prep, x_prep, nullptr, 0, nullptr, T * ks, k, wg, wu, n_experts, H, I, h, nullptr, 0, logits,
               ld_stride, norm, ids, scores, with_shared ? ks : 0};
  return gate_up(fn, a, type, type, stream);
}

extern "C" int lmoe_gemv_down_combine(const float *h, const uint32_t *ids, const float *scores, int T, int k,
                                      const uint8_t *wd, int type_d, int n_experts, int I, int H, const float *shared,
                                      const float *gate, int gate_stride, const void *residual, int rdtype,
                                      void *out, int odtype, void *stream) {
  DownArgs a{nullptr, 0, h, ids, scores, T, k, wd, type_d, n_experts, I, H, shared, gate, gate_stride, residual,
             rdtype, out, odtype};
  return down("lmoe_gemv_down_combine", a, stream);
}

extern "C" int lmoe_gemv_down_combine_prepped(const uint32_t *hprep, int has_sums, const uint32_t *ids,
                                              const float *scores, int T, int k, const uint8_t *wd, int type_d,
                                              int n_experts, int I, int H, const float *shared, const float *gate,
                                              int gate_stride, const void *residual, int rdtype, void *out,
                                              int odtype, void *stream) {
  LMOE_REQUIRE(hprep, LMOE_EINVAL, "lmoe_gemv_down_combine_prepped: null pointer");
  DownArgs a{hprep, has_sums, nullptr, ids, scores, T, k, wd, type_d, n_experts, I, H, shared, gate, gate_stride,
             residual, rdtype, out, odtype};
  return down("lmoe_gemv_down_combine_prepped", a, stream);
}

extern "C" int lmoe_gemv_gate_up_runs(const void *x, int xdtype, const uint32_t *slots, int n, int run_rows,
                                      const uint8_t *wg, const uint8_t *wu, int type_g, int type_u, int n_experts,
                                      int H, int I, float *h, void *stream) {
  return gate_up_runs(x, xdtype, slots, n, run_rows, wg, wu, type_g, type_u, n_experts, H, I, h,
                      (hipStream_t)stream);
}

extern "C" int lmoe_gemv_down_runs(const float *h, const uint32_t *slots, int n, int run_rows, const uint8_t *wd,
                                   int type_d, int n_experts, int I, int H, void *out, int odtype, void *stream) {
  return down_runs(h, slots, n, run_rows, wd, type_d, n_experts, I, H, out, odtype, (hipStream_t)stream);
}

extern "C" int lmoe_gemv_gate_up_runs_prepped(const uint32_t *x_prep, const uint32_t *slots, int n, int run_rows,
                                              const uint8_t *wg, const uint8_t *wu, int type, int n_experts, int H,
                                              int I, float *h, uint32_t *hprep, int type_d, void *stream) {
  return gate_up_runs_prepped(x_prep, slots, n, run_rows, wg, wu, type, n_experts, H, I, h, hprep, type_d,
                              (hipStream_t)stream);
}

extern "C" int lmoe_gemv_down_runs_prepped(const uint32_t *hprep, const uint32_t *slots, int n, int run_rows,
                                           const uint8_t *wd, int type_d, int n_experts, int I, int H, void *out,
                                           int odtype, void *stream) {
  return down_runs_prepped(hprep, slots, n, run_rows, wd, type_d, n_experts, I, H, out, odtype, (hipStream_t)stream);
}

extern "C" int lmoe_gemv_chain_gate_up(const void *x, int xdtype, const uint32_t *slots, int n_slots, int topk,
                                       const uint8_t *wg, const uint8_t *wu, int type, int n_experts, int H, int I,
                                       float *h, uint32_t *hprep, int type_d, void *stream) {
  return chain_gate_up(x, xdtype, slots, n_slots, topk, wg, wu, type, n_experts, H, I, h, hprep, type_d,
                       (hipStream_t)stream);
}

extern "C" int lmoe_gemv_chain_down(const uint32_t *hprep, const uint32_t *slots, int n, const uint8_t *wd,
                                    int type_d, int n_experts, int I, int H, void *out, int odtype, void *stream) {
  return down_slots(hprep, slots, n, wd, type_d, n_experts, I, H, out, odtype, (hipStream_t)stream);
}
