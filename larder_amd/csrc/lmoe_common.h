// Shared device helpers and host plumbing for the gfx950 MoE kernels.
//
// Weight "units": both block types this library reads are 0.5625 bytes a weight, so a run of 64 weights of a
// row is 36 bytes in either of them: two Q4_0 blocks (18 bytes each: f16 d, 16 bytes of nibbles), or one quarter
// of a Q4_K super-block (256 weights in 144 bytes: f16 d, f16 dmin, 12 bytes of 6-bit scales/mins, 128 bytes of
// nibbles). Row bytes are 36 * (cols / 64) for both, so one staging scheme serves both types.
//
// Dot products run on v_dot2_f32_f16: x is held as f16 pairs arranged in the order the nibbles sit in a 32-bit
// word, and a nibble q becomes the f16 value 64 + q by moving it to mantissa bits 4..7 (one shift, none for the
// nibble already there) and masking it under the exponent of 64 (0x5400): 7 operations a word of 8 nibbles. Then
// sum((64 + q) x) = 64 sum(x) + sum(q x): the block's exact sum(q x) follows from one fused multiply-add with the
// block's precomputed sum(x). Products of f16 values are exact in fp32, so the dot is an fp32-accumulated dot of
// the exact integer nibbles with the f16 activations.
//
// Prepared activations ("prep" rows): an activation row of 64 P values is kept as P units of 36 dwords, the
// layout the kernels use in LDS: dwords 0..31 the unit's f16 pairs in nibble order (xelem below), dwords 32 and 33
// the sums of the unit's two 32-value halves over the f16-rounded values, dwords 34 and 35 zero.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <stdint.h>
#include <string>

#include "../../include/larder_moe.h"

namespace lmoe {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// The value unchanged, opaque to the optimiser: per-thread arithmetic on it is redone in each iteration of an outer
// loop (a layer, a tile) instead of being hoisted out of the loop and kept live, in registers, for the whole kernel
__device__ __forceinline__ int opaque(int v) {
  asm volatile("" : "+v"(v));
  return v;
}
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}
// A float materialised as the fp32 value it is: a conversion that follows rounds that value, instead of the compiler
// merging the multiply that produced it with the conversion (v_fma_mix*_f16: one rounding in place of two)
__device__ __forceinline__ float opaque(float v) {
  asm volatile("" : "+v"(v));
  return v;
}

constexpr int XS = 36;  // dwords a prepared unit takes (32 pairs, 2 sums, 2 pad)

// ---- host-side error plumbing ----------------------------------------------------------------------------------

void set_error(const char *fmt, ...);
int fail(int code, const char *fmt, ...);
int hip_fail(hipError_t e, const char *what);

#define LMOE_REQUIRE(cond, code, ...)            \
  do {                                           \
    if (!(cond)) return ::lmoe::fail((code), __VA_ARGS__); \
  } while (0)

#define LMOE_LAUNCHED(what)                                  \
  do {                                                       \
    hipError_t _e = hipGetLastError();                       \
    if (_e != hipSuccess) return ::lmoe::hip_fail(_e, what); \
  } while (0)

// Dynamic LDS above 64 KiB must be allowed per kernel before the launch.
template <typename K>
inline int allow_lds(K kernel, size_t bytes, const char *what) {
  if (bytes <= 65536) return 0;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, int(bytes));
  return e == hipSuccess ? 0 : hip_fail(e, what);
}

// Kernel-exact timing of the library's own launches (lmoe_profile_arm / lmoe_profile_read): while armed, launch()
// brackets each kernel with a start / stop event pair recorded by the launch itself.
bool profile_next(hipEvent_t *start, hipEvent_t *stop);

// Per-workgroup phase stamps of the decode kernels (lmoe_timeline_arm): while armed, the router GEMV, the fused
// gate/up and the two-wavefront down launch their stamping forms, each workgroup writing the device's constant-rate
// wall clock into its row of 8 at each phase it reaches (0 start, 1 inputs in: logits or ids, 2 top-k done, 3 weights
// in, 4 end); a phase a workgroup does not reach stays 0. timeline_next gives a launch of n_wg workgroups its rows
// (nullptr when disarmed or full).
enum { LMOE_TL_ROUTER = 1, LMOE_TL_GATE_UP = 2, LMOE_TL_DOWN = 3 };
unsigned long long *timeline_next(int kernel, int n_wg);

template <bool TL>
__device__ __forceinline__ void tl_stamp(unsigned long long *tl, int phase) {
  if constexpr (TL) {
    if (threadIdx.x == 0)
      tl[(size_t(blockIdx.y) * gridDim.x + blockIdx.x) * 8 + phase] = (unsigned long long)wall_clock64();
  }
}

template <typename K, typename... Args>
inline void launch(K kernel, dim3 grid, dim3 block, size_t lds, hipStream_t st, Args... args) {
  hipEvent_t a, b;
  if (profile_next(&a, &b))
    hipExtLaunchKernelGGL(kernel, grid, block, uint32_t(lds), st, a, b, 0, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, lds, st, args...);
}

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned4(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }
inline bool dtype_ok(int t) { return t == LMOE_F32 || t == LMOE_F16 || t == LMOE_BF16; }
inline bool qtype_ok(int t) { return t == LMOE_Q4_0 || t == LMOE_Q4_K; }
inline int block_weights(int t) { return t == LMOE_Q4_K ? 256 : 32; }

// The general decode chain and dequant over every supported block type (anytype.hip)
bool qtype_any(int t);
int block_weights_any(int t);
int block_bytes_any(int t);
int gate_up_any(const char *fn, const void *x, int xdt, const uint32_t *slots, int n_slots, int topk,
                const uint8_t *wg, const uint8_t *wu, int tg, int tu, int n_experts, int H, int I, float *h,
                hipStream_t st);
int down_any(const char *fn, const float *h, const uint32_t *ids, const float *scores, int T, int k,
             const uint8_t *wd, int td, int n_experts, int I, int H, const float *shared, const float *gate,
             int gate_stride, const void *residual, int rdt, void *out, int odt, hipStream_t st);
int down_packed_prepped(const char *fn, int td, const uint32_t *hprep, const uint32_t *ids, const float *scores,
                        int T, int k, const uint8_t *wd, int n_experts, int I, int H, const float *shared,
                        const float *gate, int gate_stride, const void *residual, int rdt, void *out, int odt,
                        hipStream_t st);
int dequant_any(const char *fn, const uint8_t *buf, int type, int n_experts, int rows, int cols,
                const uint32_t *slots, int n, void *q, int odt, int kperm, hipStream_t st);

// ---- element loads / stores ------------------------------------------------------------------------------------

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }

// round to nearest even, NaN kept quiet
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}

__device__ __forceinline__ float load_elt(const void *p, size_t i, int dt) {
  if (dt == LMOE_F32) return static_cast<const float *>(p)[i];
  if (dt == LMOE_F16) return float(static_cast<const _Float16 *>(p)[i]);
  return bf16_to_f32(static_cast<const uint16_t *>(p)[i]);
}

__device__ __forceinline__ void store_elt(void *p, size_t i, float v, int dt) {
  if (dt == LMOE_F32)
    static_cast<float *>(p)[i] = v;
  else if (dt == LMOE_F16)
    static_cast<_Float16 *>(p)[i] = _Float16(v);
  else
    static_cast<uint16_t *>(p)[i] = f32_to_bf16(v);
}

// 8 consecutive elements at index i (16-byte aligned) as floats, and back
__device__ __forceinline__ void load8(const void *p, size_t i, int dt, float *v) {
  if (dt == LMOE_F32) {
    const float4 a = *reinterpret_cast<const float4 *>(static_cast<const float *>(p) + i);
    const float4 b = *reinterpret_cast<const float4 *>(static_cast<const float *>(p) + i + 4);
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
  } else {
    const u32x4 w = *reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(p) + i);
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (dt == LMOE_F16) {
        const h2_t hv = __builtin_bit_cast(h2_t, ws[j]);
        v[2 * j] = float(hv[0]);
        v[2 * j + 1] = float(hv[1]);
      } else {
        v[2 * j] = __uint_as_float(ws[j] << 16);
        v[2 * j + 1] = __uint_as_float(ws[j] & 0xFFFF0000u);
      }
    }
  }
}

__device__ __forceinline__ void store8(void *p, size_t i, int dt, const float *v) {
  if (dt == LMOE_F32) {
    *reinterpret_cast<float4 *>(static_cast<float *>(p) + i) = float4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<float4 *>(static_cast<float *>(p) + i + 4) = float4{v[4], v[5], v[6], v[7]};
  } else {
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (dt == LMOE_F16) {
        const h2_t h = {_Float16(v[2 * j]), _Float16(v[2 * j + 1])};
        w[j] = __builtin_bit_cast(uint32_t, h);
      } else {
        w[j] = uint32_t(f32_to_bf16(v[2 * j])) | (uint32_t(f32_to_bf16(v[2 * j + 1])) << 16);
      }
    }
    *reinterpret_cast<u32x4 *>(static_cast<uint16_t *>(p) + i) = u32x4{w[0], w[1], w[2], w[3]};
  }
}

__device__ __forceinline__ float sigmoidf_(float v) { return 1.0f / (1.0f + __expf(-v)); }

// silu(g) * u; the exponential only ever sees -|g|, so it never overflows
__device__ __forceinline__ float silu_mul(float g, float u) {
  const float e = __expf(-fabsf(g));
  const float s = g >= 0.0f ? 1.0f / (1.0f + e) : e / (1.0f + e);
  return g * s * u;
}
// The same for a result rounded to f16 right after: the hardware reciprocal (1 ulp in fp32, far below f16's
// rounding) in place of the correctly rounded division's ten-instruction sequence
__device__ __forceinline__ float silu_mul_h(float g, float u) {
  const float e = __expf(-fabsf(g));
  const float r = __builtin_amdgcn_rcpf(1.0f + e);
  const float s = g >= 0.0f ? r : e * r;
  return g * s * u;
}

// ---- cross-lane exchanges on the VALU (DPP and gfx950's permlane swaps) ------------------------------------------
//
// A dependent ds_bpermute / ds_swizzle round trip costs ~70 ns here; these stay in the vector ALU.

#define LMOE_DPP(v, ctrl) \
  __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, (v)), (ctrl), 0xF, 0xF, false))
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7 - i within 8
constexpr int kDppMirror = 0x140;      // lane i <-> 15 - i within 16
constexpr int kDppRor8 = 0x128;        // row_ror:8, lane i reads lane (i + 8) mod 16 within 16: lane i ^ 8
constexpr int kDppRor4 = 0x124;        // row_ror:4, lane i reads lane (i - 4) mod 16 within 16

// the value of lane ^ 16 / lane ^ 32
// (the swapped pair's elements are copied out as values before the cast: a bit cast of a vector element lvalue is
// lowered to element 0 by this compiler)
__device__ __forceinline__ float lane_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  const uint32_t r0 = r[0], r1 = r[1];
  return __uint_as_float((threadIdx.x & 16) ? r0 : r1);
}
__device__ __forceinline__ float lane_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  const uint32_t r0 = r[0], r1 = r[1];
  return __uint_as_float((threadIdx.x & 32) ? r0 : r1);
}

// sums over aligned groups of 8 / 16 / 64 lanes, the result in every lane of the group (fixed order: deterministic)
__device__ __forceinline__ float sum8(float v) {
  v += LMOE_DPP(v, kDppXor1);
  v += LMOE_DPP(v, kDppXor2);
  v += LMOE_DPP(v, kDppHalfMirror);
  return v;
}
__device__ __forceinline__ float sum16(float v) {
  v = sum8(v);
  return v + LMOE_DPP(v, kDppMirror);
}
// lane l's value (wave-uniform result)
__device__ __forceinline__ float lane_value(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
// The cross-row steps read the four rows' totals with readlane (scalar results, no lane exchange round trip);
// the association, (row 0 + row 1) + (row 2 + row 3), is the pairwise tree of a butterfly, so every lane gets the
// same bits a butterfly would give it.
__device__ __forceinline__ float wave_sum(float v) {
  v = sum16(v);
  return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, LMOE_DPP(v, kDppXor1));
  v = fmaxf(v, LMOE_DPP(v, kDppXor2));
  v = fmaxf(v, LMOE_DPP(v, kDppHalfMirror));
  v = fmaxf(v, LMOE_DPP(v, kDppMirror));
  return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

// ---- top-k over a wavefront -------------------------------------------------------------------------------

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  v = min(v, uint32_t(__builtin_amdgcn_update_dpp(0, int(v), kDppXor1, 0xF, 0xF, false)));
  v = min(v, uint32_t(__builtin_amdgcn_update_dpp(0, int(v), kDppXor2, 0xF, 0xF, false)));
  v = min(v, uint32_t(__builtin_amdgcn_update_dpp(0, int(v), kDppHalfMirror, 0xF, 0xF, false)));
  v = min(v, uint32_t(__builtin_amdgcn_update_dpp(0, int(v), kDppMirror, 0xF, 0xF, false)));
  v = min(v, __builtin_bit_cast(uint32_t, lane_xor16(__builtin_bit_cast(float, v))));
  v = min(v, __builtin_bit_cast(uint32_t, lane_xor32(__builtin_bit_cast(float, v))));
  return v;
}

// Order-preserving key of a logit: a larger logit has a larger key; -0 is folded into +0 so the two tie.
__device__ __forceinline__ uint32_t logit_key(float f) {
  const uint32_t u = f == 0.0f ? 0u : __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_logit(uint32_t key) {
  return __uint_as_float((key & 0x80000000u) ? (key & 0x7FFFFFFFu) : ~key);
}

// One wavefront, a token's logits v[j] = row[lane + 64 j] (j < NPL, E <= 64 NPL): lane r < k gets the rank-r pick
// (largest logit first, equal logits by lower expert index) in *id_out and its softmax probability (max-subtracted,
// fp32), renormalised over the k picks in rank order when norm, in *score_out (SCORES false: ids only, score_out
// untouched). lds: 64 dwords of this wavefront's LDS, 16-byte aligned. No step loops over k:
//   1. thr = the k-th largest key, by a 32-step bitwise search on the scalar unit: bit b stays set when at least k
//      keys are >= the prefix (one compare a value and a ballot popcount a step);
//   2. the picks are the keys above thr, then the lowest-index keys equal to thr up to k, compacted into LDS in
//      index order (a count other than k, impossible with the right threshold, sets every id to 0xFFFFFFFF);
//   3. each pick's rank is the number of picks ahead of it, then a lane permute puts rank r in lane r.
// SCORES false: only the pick of rank `want` (wavefront-uniform) is wanted; *id_out is that id in every lane, found
// by a ballot over the ranks instead of the permute to rank order.
template <int NPL, bool SCORES = true>
__device__ __forceinline__ void topk_wave(const float *v, int E, int k, int norm, uint32_t *lds, uint32_t *id_out,
                                          float *score_out, int want = 0) {
  const int lane = threadIdx.x & 63;
  uint32_t key[NPL];
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const bool ok = lane + 64 * j < E;
    key[j] = ok ? logit_key(v[j]) : 0u;  // every real key is above 0 (-inf has key 0x007FFFFF)
    if (ok) m = fmaxf(m, v[j]);
  }
  float s = 0.0f;
  if (SCORES) {  // the softmax terms only where the scores are wanted
    m = wave_max(m);
#pragma unroll
    for (int j = 0; j < NPL; ++j)
      if (lane + 64 * j < E) s += __expf(v[j] - m);
    s = wave_sum(s);
  }
  // 1. the k-th largest key, or a threshold with the same picks: bit b stays set while at least k keys are at or
  // above the prefix; once exactly k are, no lower bit changes which keys those are (every later threshold lies
  // between the prefix and the k-th key), so the search stops there. Ties at the k-th key run all 32 steps.
  uint32_t thr = 0;
  for (int b = 31; b >= 0; --b) {
    const uint32_t cand = thr | (1u << b);
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < NPL; ++j) cnt += __popcll(__ballot(key[j] >= cand));
    if (cnt >= k) {  // cnt is wavefront-uniform: a scalar branch
      thr = cand;
      if (cnt == k) break;
    }
  }
  // 2. the picks, compacted in index order (expert lane + 64 j: j major, then lane)
  const uint64_t below = (uint64_t(1) << lane) - 1;
  int n_gt = 0;
#pragma unroll
  for (int j = 0; j < NPL; ++j) n_gt += __popcll(__ballot(key[j] > thr));
  const int need = k - n_gt;  // ties at thr picked, lowest index first (none when the search stopped early)
  int eq_before = 0, sel_before = 0;
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const uint64_t eq = __ballot(key[j] == thr);
    const bool tie = (eq >> lane) & 1u;
    const bool sel = key[j] > thr || (tie && eq_before + __popcll(eq & below) < need);
    const uint64_t selm = __ballot(sel);
    const int pos = sel_before + __popcll(selm & below);
    if (sel && pos < 32) {  // at most k <= 32 picks; the bound keeps every write inside this wavefront's 64 dwords
      lds[pos] = key[j];
      lds[32 + pos] = uint32_t(lane + 64 * j);
    }
    eq_before += __popcll(eq);
    sel_before += __popcll(selm);
  }
  // exactly k picks by construction (emulated on the CPU in tests/emul/topk_wave.cpp); any other count would mean a
  // wrong threshold, and then every id of the token is 0xFFFFFFFF (no expert: zero rows downstream, and a mismatch
  // in every parity test) instead of a silently truncated pick list
  const bool bad = sel_before != k;
  __builtin_amdgcn_wave_barrier();
  // 3. ranks, then rank order
  uint32_t my_key = 0, my_idx = 0;
  int rank = lane;
  if (lane < k) {
    my_key = lds[lane];
    my_idx = lds[32 + lane];
    rank = 0;
    const u32x4 *k4 = reinterpret_cast<const u32x4 *>(lds), *i4 = reinterpret_cast<const u32x4 *>(lds + 32);
    for (int o = 0; o < k; o += 8) {  // 8 picks a step, two 16-byte broadcast reads each of keys and ids
      const u32x4 ka = k4[o / 4], kb = k4[o / 4 + 1], ia = i4[o / 4], ib = i4[o / 4 + 1];
      const uint32_t ko[8] = {ka.x, ka.y, ka.z, ka.w, kb.x, kb.y, kb.z, kb.w};
      const uint32_t io[8] = {ia.x, ia.y, ia.z, ia.w, ib.x, ib.y, ib.z, ib.w};
#pragma unroll
      for (int q = 0; q < 8; ++q)
        rank += (o + q < k && (ko[q] > my_key || (ko[q] == my_key && io[q] < my_idx))) ? 1 : 0;
    }
  }
  if (!SCORES) {  // the lane holding rank `want` (one of the first k: ranks are distinct)
    const uint64_t hit = __ballot(lane < k && rank == want);
    const uint32_t id = uint32_t(__builtin_amdgcn_readlane(int(my_idx), hit ? __builtin_ctzll(hit) : 0));
    *id_out = bad || !hit ? 0xFFFFFFFFu : id;
    return;
  }
  __builtin_amdgcn_wave_barrier();
  const int dst = (rank & 63) * 4;
  const uint32_t id = uint32_t(__builtin_amdgcn_ds_permute(dst, int(my_idx)));
  *id_out = bad ? 0xFFFFFFFFu : id;
  const uint32_t kr = uint32_t(__builtin_amdgcn_ds_permute(dst, int(my_key)));
  float mine = lane < k ? __expf(key_logit(kr) - m) / s : 0.0f;
  if (norm) {
    float tot = 0.0f;  // the k picked probabilities summed in rank order
    for (int r = 0; r < k; ++r)
      tot += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mine), r));
    mine = mine / tot;
  }
  *score_out = mine;
}

// The expert of rank `want` (0-based; larger logit first, equal logits by lower index) of a token's logits
// v[j] = row[lane + 64 j] (j < NPL, E <= 64 NPL), in every lane: the pick topk_wave<NPL, false> returns for that rank,
// without its compaction and ranking (no LDS). The one-bit search of topk_wave for the (want + 1)-th largest key:
//   * stopped at a prefix with exactly want + 1 keys at or above it, those keys are ranks 0 .. want, so rank want is
//     the smallest of them, the highest index among equal ones;
//   * run to the end, the prefix is the (want + 1)-th largest key itself, and rank want is the
//     (want + 1 - #keys above it)-th lowest index holding it.
// Emulated on the CPU against the oracle on tie-heavy rows (tests/emul/topk_wave.cpp, rank_pick). 0xFFFFFFFF when no
// key qualifies (E <= want).
template <int NPL>
__device__ __forceinline__ uint32_t rank_pick_wave(const float *v, int E, int want) {
  const int lane = threadIdx.x & 63;
  uint32_t key[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) key[j] = lane + 64 * j < E ? logit_key(v[j]) : 0u;
  const int need = want + 1;
  uint32_t thr = 0;
  bool exact = false;
#pragma unroll  // straight-line code: each candidate an immediate, the prefix in a scalar register
  for (int b = 31; b >= 0; --b) {
    const uint32_t cand = thr | (1u << b);
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < NPL; ++j) cnt += __popcll(__ballot(key[j] >= cand));
    if (cnt >= need) {  // wavefront-uniform: a scalar branch
      thr = cand;
      if (cnt == need) {
        exact = true;
        break;
      }
    }
  }
  if (exact) {
    uint32_t m = 0xFFFFFFFFu;
#pragma unroll
    for (int j = 0; j < NPL; ++j) m = min(m, key[j] >= thr ? key[j] : 0xFFFFFFFFu);
    m = wave_min_u32(m);
#pragma unroll
    for (int j = NPL - 1; j >= 0; --j) {
      const uint64_t eq = __ballot(key[j] == m);
      if (eq) return uint32_t(64 * j + 63 - __builtin_clzll(eq));
    }
    return 0xFFFFFFFFu;
  }
  int n_gt = 0;
#pragma unroll
  for (int j = 0; j < NPL; ++j) n_gt += __popcll(__ballot(key[j] > thr));
  int rem = need - n_gt;  // >= 1: fewer than want + 1 keys lie above the (want + 1)-th largest
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    uint64_t eq = __ballot(key[j] == thr);
    const int c = __popcll(eq);
    if (rem <= c) {
      for (int i = 1; i < rem; ++i) eq &= eq - 1;  // clear the rem - 1 lowest holders
      return uint32_t(64 * j + __builtin_ctzll(eq));
    }
    rem -= c;
  }
  return 0xFFFFFFFFu;
}

// Entries of ck[f0, f0 + 2 N) (composite keys, 16-byte aligned) above `me`. Composite key: order-preserving logit
// key in the high half, 0xFFFFFFFF - expert in the low half, so a larger composite is the better pick (larger logit,
// or equal logit and lower index) and no two experts tie; 0 pads an empty slot below every expert.
template <int N>
__device__ __forceinline__ int count_above(const uint64_t *ck, int f0, uint64_t me) {
  typedef uint64_t u64x2 __attribute__((ext_vector_type(2)));
  const u64x2 *p = reinterpret_cast<const u64x2 *>(ck + f0);
  int c = 0;
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const u64x2 v = p[j];
    const uint64_t v0 = v.x, v1 = v.y;
    c += (v0 > me ? 1 : 0) + (v1 > me ? 1 : 0);
  }
  return c;
}

// ---- top-k of one token by a 256-thread workgroup ------------------------------------------------------------

constexpr int kRankMaxE = 512;
constexpr int kRankMaxK = 16;

struct RankScratch {
  float vals[kRankMaxE + 16];
  uint64_t ck[kRankMaxE];
  uint64_t surv[8 * kRankMaxK];
  uint32_t cnt[128 * 8];
  uint32_t pick[kRankMaxK];
  float praw[kRankMaxK];
  float red[4];
};

// The top k of vals[0, E) (LDS) by the 256 threads of the workgroup: composite keys (logit key above, 0xFFFFFFFF -
// expert below: no ties, lower index first among equal logits); E > 128: the best k of each 64-candidate chunk
// survive; the survivors' ranks are the sums of counts over 8 groups of 16. Leaves ids in s.pick, and returns in
// threads r < k the softmax probability of pick r (max subtracted, fp32; renormalised in rank order when norm).
__device__ __forceinline__ float rank256(RankScratch &s, int E, int k, int norm, int tid) {
  typedef uint64_t u64x2 __attribute__((ext_vector_type(2)));
  uint64_t mine[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int e = tid + 256 * j;
    mine[j] = e < E ? (uint64_t(logit_key(s.vals[e])) << 32) | (0xFFFFFFFFu - uint32_t(e)) : 0u;
    s.ck[e] = mine[j];
  }
  if (tid < 8 * kRankMaxK) s.surv[tid] = 0u;
  __syncthreads();
  const uint64_t *set = s.ck;
  if (E > 128) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int e = tid + 256 * j;
      const int c = count_above<32>(s.ck, e & ~63, mine[j]);
      if (e < E && c < k) s.surv[(e >> 6) * k + c] = mine[j];
    }
    __syncthreads();
    set = s.surv;
  }
  {
    const int g = tid & 31, q = tid >> 5;
    const u64x2 *p16 = reinterpret_cast<const u64x2 *>(set + 16 * q);
    uint64_t o[16];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const u64x2 v = p16[j];
      o[2 * j] = v.x;
      o[2 * j + 1] = v.y;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint64_t me = set[g + 32 * i];
      int c = 0;
#pragma unroll
      for (int j = 0; j < 16; ++j) c += o[j] > me ? 1 : 0;
      s.cnt[(g + 32 * i) * 8 + q] = uint32_t(c);
    }
  }
  __syncthreads();
  if (tid < 128 && set[tid] != 0u) {
    const u32x4 *c4 = reinterpret_cast<const u32x4 *>(s.cnt + 8 * tid);
    const u32x4 a = c4[0], b = c4[1];
    const uint32_t r = a.x + a.y + a.z + a.w + b.x + b.y + b.z + b.w;
    if (r < uint32_t(k)) s.pick[r] = 0xFFFFFFFFu - uint32_t(set[tid]);
  }
  __syncthreads();
  // softmax denominator: this thread's two terms, a wavefront tree, the four wavefronts left to right
  const float m = s.vals[s.pick[0]];
  float term = 0.0f;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int e = tid + 256 * j;
    if (e < E) term += __expf(s.vals[e] - m);
  }
  term = wave_sum(term);
  if ((tid & 63) == 0) s.red[tid >> 6] = term;
  __syncthreads();
  const float tot = ((s.red[0] + s.red[1]) + s.red[2]) + s.red[3];
  float p = 0.0f;
  if (tid < k) {
    p = __expf(s.vals[s.pick[tid]] - m) / tot;
    s.praw[tid] = p;
  }
  __syncthreads();
  if (tid < k && norm) {
    float sum = 0.0f;  // the k probabilities in rank order
    for (int r = 0; r < k; ++r) sum += s.praw[r];
    p = p / sum;
  }
  return p;
}

// ---- nibble words -> f16 pairs ----------------------------------------------------------------------------------

// (t & 0x00F000F0) | 0x54005400 in one v_and_or_b32. With both constants as literals the compiler splits it into an
// and and an or (the fused form takes at most one literal or scalar operand on gfx9), so the mask comes from a
// vector register: a one-instruction asm moves it there (not volatile, so every call shares one), and the and-or
// stays plain code the scheduler sees through. Writing the whole v_and_or_b32 as asm instead cost 190 VGPRs
// against 111 in the Q4_K gate/up kernel at H = 4096 (occupancy 2 waves a SIMD instead of 3).
__device__ __forceinline__ uint32_t and_or_nib(uint32_t t) {
  uint32_t m;
  asm("v_mov_b32 %0, 0xf000f0" : "=v"(m));
  return (t & m) | 0x54005400u;
}

// The f16 pair (64 + a, 64 + b) from nibbles a, b sitting at bits [s, s+4) and [s+16, s+20) of w (0 <= s <= 12).
template <int S>
__device__ __forceinline__ uint32_t nib_pair(uint32_t w) {
  const uint32_t t = S == 4 ? w : (S < 4 ? (w << (4 - S)) : (w >> (S - 4)));
  return and_or_nib(t);
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, a), __builtin_bit_cast(h2_t, b), c, false);
}

// sum((64 + q) x) over the 8 nibbles of qs word w against x pairs xp[0..3] =
// (x[j], x[j+2]), (x[j+H], x[j+H+2]), (x[j+1], x[j+3]), (x[j+H+1], x[j+H+3]) where the word's low nibbles are
// weights j..j+3 and its high nibbles weights j+H..j+H+3 (H = 16 for Q4_0, 32 for Q4_K).
__device__ __forceinline__ float word_dot(uint32_t w, const uint32_t *xp, float acc) {
  acc = dot2(nib_pair<0>(w), xp[0], acc);
  acc = dot2(nib_pair<4>(w), xp[1], acc);
  acc = dot2(nib_pair<8>(w), xp[2], acc);
  acc = dot2(nib_pair<12>(w), xp[3], acc);
  return acc;
}

__device__ __forceinline__ float half_lo(uint32_t w) { return float(__builtin_bit_cast(h2_t, w)[0]); }
__device__ __forceinline__ float half_hi(uint32_t w) { return float(__builtin_bit_cast(h2_t, w)[1]); }

// 8 values at element index i of a row of dtype dt, from one or two 16-byte chunks already loaded
__device__ __forceinline__ void unpack8(const u32x4 &a, const u32x4 &b, int dt, float *v) {
  const uint32_t u[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  if (dt == LMOE_F32) {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = __uint_as_float(u[e]);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = dt == LMOE_F16 ? half_lo(u[e]) : __uint_as_float(u[e] << 16);
      v[2 * e + 1] = dt == LMOE_F16 ? half_hi(u[e]) : __uint_as_float(u[e] & 0xFFFF0000u);
    }
  }
}

// Position of natural element n (a multiple of 4) of a row in the GEMMs' K order: within each 32-wide block,
// group n4 = (n % 32) / 4 sits at 8 n4 (n4 < 4) or 8 (n4 - 4) + 4
__device__ __forceinline__ int kperm4(int n) {
  const int n4 = (n & 31) >> 2;
  return (n & ~31) | (n4 < 4 ? 8 * n4 : 8 * (n4 - 4) + 4);
}

// Elements [2048 block, +2048) of x (n of them, dtype dt, n % 32 == 0, 16-byte aligned) to f16 in the K order: 8 a
// thread, one 16-byte load and two 8-byte stores (a 4-element group keeps its neighbours within the 32-block).
__device__ __forceinline__ void to_f16_kperm(int block, const void *x, int dt, long long n, _Float16 *out) {
  const long long i0 = (static_cast<long long>(block) * 256 + threadIdx.x) * 8;
  if (i0 >= n) return;
  float v[8];
  load8(x, size_t(i0), dt, v);
  const long long b = i0 & ~31ll;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const h2_t p0 = {_Float16(v[4 * h]), _Float16(v[4 * h + 1])}, p1 = {_Float16(v[4 * h + 2]), _Float16(v[4 * h + 3])};
    *reinterpret_cast<u32x2 *>(out + b + kperm4(int(i0 & 31) + 4 * h)) =
        u32x2{__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1)};
  }
}

// ---- x arrangement ----------------------------------------------------------------------------------------------
//
// A unit of 64 weights takes 32 dwords of x pairs, arranged so that word i of a block's (or sub-block pair's)
// nibbles meets the four pairs word_dot() expects.
//
// Q4_0 block (32 weights): qs word i (i = 0..3) holds weights 4i..4i+3 (low) and 16+4i..16+4i+3 (high).
// Q4_K sub-block pair (64 weights): qs word i (i = 0..7) holds weights 4i..4i+3 of sub-block 2c (low nibbles) and
//   the same of sub-block 2c+1 (high nibbles), i.e. unit weights 4i.. and 32+4i...
// Both are "word i covers weights {4i..4i+3} + {H+4i..H+4i+3}" over a span of 2H weights, H = 16 (two spans a
// unit) or 32 (one span). A span of 2H weights fills H dwords. Dword dw of the unit, half h, holds weight
// span * 2H + hi * H + 4i + r with span = dw / H, i = (dw mod H) / 4, s = dw mod 4 the pair slot (A, B, C, D =
// 0..3: r even / odd, low / high nibbles), hi = s & 1 and r = (s >> 1) + 2h.
__device__ __forceinline__ int xelem(int dw, int h, int H) {
  const int span = dw / H, i = (dw % H) >> 2, s = dw & 3;
  return span * 2 * H + (s & 1) * H + 4 * i + (s >> 1) + 2 * h;
}
// the inverse: unit weight e -> (dword, half)
__device__ __forceinline__ void xslot(int e, int H, int *dw, int *half) {
  const int span = e / (2 * H), f = e % (2 * H), hi = f >= H ? 1 : 0, g = f % H, i = g >> 2, r = g & 3;
  *dw = span * H + 4 * i + 2 * (r & 1) + hi;
  *half = r >> 1;
}

// qs word i of Q4_K sub-block pair c from the 12-byte scale field words s0, s1, s2: (sc, m) of sub-blocks 2c and
// 2c + 1, ggml's get_scale_min_k4 (gguf_ref.py:253-258): j < 4: sc = q[j] & 63, m = q[j+4] & 63; j >= 4:
// sc = (q[j+4] & 15) | (q[j-4] >> 6) << 4, m = (q[j+4] >> 4) | (q[j] >> 6) << 4.
__device__ __forceinline__ uint32_t byte_of(uint32_t s0, uint32_t s1, uint32_t s2, int j) {
  const uint32_t w = j < 4 ? s0 : (j < 8 ? s1 : s2);
  return (w >> (8 * (j & 3))) & 0xFFu;
}
__device__ __forceinline__ void k4_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j, float *sc, float *m) {
  uint32_t a, b;
  if (j < 4) {
    a = byte_of(s0, s1, s2, j) & 63u;
    b = byte_of(s0, s1, s2, j + 4) & 63u;
  } else {
    const uint32_t q8 = byte_of(s0, s1, s2, j + 4);
    a = (q8 & 15u) | ((byte_of(s0, s1, s2, j - 4) >> 6) << 4);
    b = (q8 >> 4) | ((byte_of(s0, s1, s2, j) >> 6) << 4);
  }
  *sc = float(a);
  *m = float(b);
}

// One 64-weight unit's dot with x, given the unit's 36 bytes as 9 dwords u[0..8] (Q4_0: two blocks; the unit
// starts 4-byte aligned) or, for Q4_K, the super-block header h[0..3] and the 8 qs words q[0..7] of pair c.
// xp: the unit's 32 x-pair dwords; sx0/sx1: sum of x over the unit's first / last 32 weights.
__device__ __forceinline__ float unit_dot_q4_0(const uint32_t *u, const uint32_t *xp, float sx0, float sx1) {
  // block A: d = low half of u0, qs bytes at unit bytes 2..17 -> realign by 2 bytes
  float a = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) a = word_dot(__builtin_amdgcn_alignbyte(u[i + 1], u[i], 2), xp + 4 * i, a);
  // block B: d = high half of u4, qs = u5..u8
  float b = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) b = word_dot(u[5 + i], xp + 16 + 4 * i, b);
  const float dA = half_lo(u[0]), dB = half_hi(u[4]);
  // sum((q - 8) x) = sum((64 + q) x) - 72 sum(x)
  return dA * fmaf(-72.0f, sx0, a) + dB * fmaf(-72.0f, sx1, b);
}

__device__ __forceinline__ float unit_dot_q4_k(const uint32_t *hdr, const uint32_t *q, int c, const uint32_t *xp,
                                               float sx0, float sx1) {
  float a = 0.0f, b = 0.0f;
  // word i: low nibbles -> sub-block 2c weights 4i..4i+3, high -> sub-block 2c+1; word_dot pairs (A, B, C, D)
  // are (lo 4i/4i+2, hi 4i/4i+2, lo 4i+1/4i+3, hi 4i+1/4i+3): low-nibble pairs feed a, high-nibble pairs b.
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t w = q[i];
    a = dot2(nib_pair<0>(w), xp[4 * i + 0], a);
    b = dot2(nib_pair<4>(w), xp[4 * i + 1], b);
    a = dot2(nib_pair<8>(w), xp[4 * i + 2], a);
    b = dot2(nib_pair<12>(w), xp[4 * i + 3], b);
  }
  const float d = half_lo(hdr[0]), dmin = half_hi(hdr[0]);
  float sc0, m0, sc1, m1;
  k4_scale_min(hdr[1], hdr[2], hdr[3], 2 * c, &sc0, &m0);
  k4_scale_min(hdr[1], hdr[2], hdr[3], 2 * c + 1, &sc1, &m1);
  // w = (d sc) q - (dmin m): sum(w x) = (d sc) (sum((64 + q) x) - 64 sum(x)) - (dmin m) sum(x)
  const float ra = (d * sc0) * fmaf(-64.0f, sx0, a) - (dmin * m0) * sx0;
  const float rb = (d * sc1) * fmaf(-64.0f, sx1, b) - (dmin * m1) * sx1;
  return ra + rb;
}

// The dot of unit p of a staged row (9 P dwords) with an activation unit held in registers (pairs xv, sums sx0 / sx1).
template <int TQ>
__device__ __forceinline__ float row_unit_dot_r(const uint32_t *row, int p, const uint32_t *xv, float sx0, float sx1) {
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

// sum over the aligned group of P lanes (P = 32 or 64), the result in every lane of the group
template <int P>
__device__ __forceinline__ float group_sum(float v) {
  if (P == 64) return wave_sum(v);
  v = sum16(v);
  const float g0 = lane_value(v, 0) + lane_value(v, 16), g1 = lane_value(v, 32) + lane_value(v, 48);
  return (threadIdx.x & 32) ? g1 : g0;
}

// ---- preparing activation rows -----------------------------------------------------------------------------------

// Unit dword (p, dw) of a prepared row for block type TQ, from an element reader ld(i) over the row's 64 P values.
template <int TQ, typename Ld>
__device__ __forceinline__ uint32_t prep_dword(Ld ld, int p, int dw) {
  constexpr int H = TQ == LMOE_Q4_K ? 32 : 16;
  if (dw < 32) {
    const h2_t v = {_Float16(ld(64 * p + xelem(dw, 0, H))), _Float16(ld(64 * p + xelem(dw, 1, H)))};
    return __builtin_bit_cast(uint32_t, v);
  }
  if (dw < 34) {  // the 32 values read first, then added in element order
    float v[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) v[j] = float(_Float16(ld(64 * p + 32 * (dw - 32) + j)));
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) s += v[j];
    return __builtin_bit_cast(uint32_t, s);
  }
  return 0u;
}

}  // namespace lmoe
