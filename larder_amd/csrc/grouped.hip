// Grouped expert GEMMs on the matrix cores, for prefill and batched decode: rows grouped by expert on the device
// (lmoe_group_rows), then one 128 x 256 output tile per (expert, m-tile, n-tile) through v_mfma_f32_16x16x32_f16.
//
// The reference's prefill path ("dense", gguf_experts.py:698-722) dequantizes up to 8 experts at a time to f16 in
// HBM (DEQ_SRC, :529-539) and runs MLX gather_mm on host-sorted rows. Here no weight is dequantized to HBM and the
// host never waits:
//   * the work list (expert << 20 | m-tile) and its length come from the grouping kernel; the 1-D grid is sized
//     for the most tiles R rows can make and workgroups past the device-side count exit at once. Workgroups are
//     dealt round-robin over the 8 XCDs, so the linear id is remapped to give each XCD one contiguous stretch of
//     work (neighbouring n-tiles of one m-tile share A rows and the expert's weights in that XCD's L2);
//   * four wavefronts, each 128 rows x 64 features (8 x 4 accumulators of 16 x 16). The A tile (128 rows x 64 of
//     K, f16: x gathered through the grouped order, or the grouped h rows) goes through LDS, shared by the four;
//     the weights do not: each K step, thread t loads the Q4 unit (64 weights) of tile feature t and repacks it
//     into LDS as one nibble word per (MFMA K slice, lane group) plus its scales, so an MFMA lane reads one word
//     and one scale word and decodes its 8 weights to f16 in registers (w = ((1024 + q) - 1032) d for Q4_0,
//     ((1024 + q) - 1024) (d sc) - dmin m for Q4_K), straight into the MFMA's weight operand. LDS then carries
//     the A tile (16 KB written, 64 KB read a step) and 10 KB of packed weights instead of a 32 KB f16 weight
//     tile written and read twice;
//   * the global loads of step k + 1 are in flight while step k's MFMAs run; one barrier a step;
//   * the weights are the MFMA's first operand, so each lane ends with 4 consecutive output features of one row;
//     gate/up tiles hold 128 gate and 128 up features (a wavefront: 32 of each, the same ones), SwiGLU happens in
//     registers and h leaves as f16 in grouped row order. Down writes y [R][H] (f16 or f32) in grouped order.
// Operands are f16 with fp32 accumulation. A single rounding of (q - 8) d to f16 keeps the layer well inside the
// 2e-3 relative L2 bar; bf16 operands would not.
#include <type_traits>

#include "lmoe_common.h"

namespace lmoe {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int GM = 128;  // rows a tile (the grouping kernel's bm)
constexpr int GN = 256;  // weight rows a tile (gate/up: 128 gate + 128 up features; down: 256 outputs)
constexpr int GK = 64;   // K a step (one 64-weight unit of every weight row)
constexpr int kThreads = 256;
constexpr int kWp = 10;  // LDS words a weight row a step: 8 nibble words, 2 scale words
constexpr int kTileMask = (1 << 20) - 1;

enum { MODE_GATE_UP = 0, MODE_DOWN = 1 };

template <int N>
using IC = std::integral_constant<int, N>;

// 16-byte chunk c (0..7) of A row r in a stage: rows are 128 bytes, chunks XOR-swizzled by the row's low 3 bits
__device__ __forceinline__ int achunk(int r, int c) { return r * 8 + (c ^ (r & 7)); }

// two f16 (1024 + q) from a byte-wise masked word: {q0, q1} or {q2, q3}
__device__ __forceinline__ uint32_t magic_pair(uint32_t nib, uint32_t sel) {
  return __builtin_amdgcn_perm(0x64646464u, nib, sel);
}
constexpr uint32_t kSel01 = 0x04010400u, kSel23 = 0x04030402u;

// Raw words of one weight row's unit kk: Q4_0 the unit's 9 words (two 18-byte blocks); Q4_K the super-block's
// header (d, dmin, 12 scale bytes) and the 8 qs words of sub-block pair kk % 4
template <int TB>
struct RawW {
  static constexpr int N = TB == LMOE_Q4_0 ? 9 : 12;
};

template <int TB>
__device__ __forceinline__ void load_w(const uint8_t *wrow, int kk, uint32_t *r) {
  if (TB == LMOE_Q4_0) {
    const uint32_t *u = reinterpret_cast<const uint32_t *>(wrow + size_t(kk) * 36);
#pragma unroll
    for (int i = 0; i < 9; ++i) r[i] = u[i];
  } else {
    const uint32_t *sb = reinterpret_cast<const uint32_t *>(wrow + size_t(kk >> 2) * 144);
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = sb[i];
#pragma unroll
    for (int i = 0; i < 8; ++i) r[4 + i] = sb[4 + 8 * (kk & 3) + i];
  }
}

// 8 nibbles of bytes j (low nibble) and j + 4 (high nibble) of a byte group: weights 0..3 / 4..7 of an MFMA lane
__device__ __forceinline__ uint32_t pack_lo(uint32_t w0, uint32_t w1) {
  return (w0 & 0x0F0F0F0Fu) | ((w1 & 0x0F0F0F0Fu) << 4);
}
__device__ __forceinline__ uint32_t pack_hi(uint32_t w0, uint32_t w1) {
  return ((w0 >> 4) & 0x0F0F0F0Fu) | (w1 & 0xF0F0F0F0u);
}

// A unit's packed words: o[4 ks + g] holds the weights 32 ks + 8 g .. + 7 of the unit (MFMA K slice ks, lane group
// g) as nibbles, o[8 + ks] the slice's scales. Q4_0 slice ks is block ks (qs byte i: weight i low, i + 16 high):
// lane group g reads bytes 8 (g % 2) .. + 7, low nibbles for g < 2; scales {d0, d1} in o[8]. Q4_K slice ks is
// sub-block 2 (kk % 4) + ks, the low (ks = 0) or high (ks = 1) nibbles of the pair's bytes 8 g .. 8 g + 7;
// o[8 + ks] = {f16(d sc), f16(dmin m)} of that sub-block (get_scale_min_k4, gguf_ref.py:253-258).
template <int TB>
__device__ __forceinline__ void pack_w(const uint32_t *r, int kk, uint32_t *o) {
  if (TB == LMOE_Q4_0) {
    uint32_t q0[4];  // block 0's qs start at unit byte 2
#pragma unroll
    for (int i = 0; i < 4; ++i) q0[i] = __builtin_amdgcn_alignbyte(r[i + 1], r[i], 2);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const uint32_t *q = ks ? r + 5 : q0;
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        o[4 * ks + b] = pack_lo(q[2 * b], q[2 * b + 1]);
        o[4 * ks + 2 + b] = pack_hi(q[2 * b], q[2 * b + 1]);
      }
    }
    o[8] = (r[0] & 0xFFFFu) | (r[4] & 0xFFFF0000u);
    o[9] = 0u;
  } else {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      o[g] = pack_lo(r[4 + 2 * g], r[5 + 2 * g]);
      o[4 + g] = pack_hi(r[4 + 2 * g], r[5 + 2 * g]);
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      float sc, mn;
      k4_scale_min(r[1], r[2], r[3], 2 * (kk & 3) + ks, &sc, &mn);
      const h2_t v = {_Float16(half_lo(r[0]) * sc), _Float16(half_hi(r[0]) * mn)};
      o[8 + ks] = __builtin_bit_cast(uint32_t, v);
    }
  }
}

// An MFMA lane's 8 f16 weights from its packed word and the slice's scale word
template <int TB>
__device__ __forceinline__ half8 decode8(uint32_t x, uint32_t sw, int ks) {
  const uint32_t lo = x & 0x0F0F0F0Fu, hi = (x >> 4) & 0x0F0F0F0Fu;
  const h2_t p[4] = {__builtin_bit_cast(h2_t, magic_pair(lo, kSel01)), __builtin_bit_cast(h2_t, magic_pair(lo, kSel23)),
                     __builtin_bit_cast(h2_t, magic_pair(hi, kSel01)), __builtin_bit_cast(h2_t, magic_pair(hi, kSel23))};
  h2_t bias, scale, sub;
  if (TB == LMOE_Q4_0) {
    const _Float16 d = __builtin_bit_cast(h2_t, sw)[ks];
    bias = h2_t{_Float16(1032.0f), _Float16(1032.0f)};
    scale = h2_t{d, d};
    sub = h2_t{_Float16(0.0f), _Float16(0.0f)};
  } else {
    const h2_t v = __builtin_bit_cast(h2_t, sw);
    bias = h2_t{_Float16(1024.0f), _Float16(1024.0f)};
    scale = h2_t{v[0], v[0]};
    sub = h2_t{v[1], v[1]};
  }
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = __builtin_bit_cast(uint32_t, (p[i] - bias) * scale - sub);
  return __builtin_bit_cast(half8, u32x4{o[0], o[1], o[2], o[3]});
}

// Grid: n_ntile * max_tiles workgroups of 256 threads (1-D), two a CU. GATE_UP: n-tile j covers intermediate
// features 128 j .. 128 j + 127 (tile features 0..127 their gate rows, 128..255 their up rows), K = H, A rows
// x[order[p] / topk], out h [R][I] f16. DOWN: n-tile j covers output features 256 j .., K = I, A rows h[p], out
// y [R][H] in odt (F16 / F32).
template <int MODE, int TB>
__global__ void __launch_bounds__(kThreads, 2)
k_grouped(const _Float16 *a_src, int topk, const uint32_t *order, const uint32_t *offsets, const uint32_t *tiles,
          const uint32_t *n_tiles, int n_ntile, const uint8_t *w0, const uint8_t *w1, int K, int n_rows, void *out,
          int ldo, int odt) {
  // A tile: rows of 64 halves = 8 swizzled 16-byte chunks; packed weights: kWp words a tile feature; 2 stages each
  __shared__ __attribute__((aligned(16))) u32x4 As[2][GM * 8];
  __shared__ __attribute__((aligned(16))) uint32_t Wp[2][GN * kWp];

  // XCD-aware remap: workgroup `wid` runs on XCD wid % 8; XCD x gets logical work [start_x, start_x + count_x)
  const uint32_t W = n_tiles[0] * uint32_t(n_ntile);
  const uint32_t wid = blockIdx.x;
  if (wid >= W) return;
  const uint32_t q8 = W >> 3, r8 = W & 7, xcd = wid & 7;
  const uint32_t logical = xcd * q8 + min(xcd, r8) + (wid >> 3);
  const uint32_t tile = tiles[logical / uint32_t(n_ntile)];
  const int nt = int(logical % uint32_t(n_ntile));
  const int e = int(tile >> 20);
  const int row0 = int(offsets[e]) + int(tile & kTileMask) * GM;
  const int rows = min(GM, int(offsets[e + 1]) - row0);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fr = lane & 15, g = lane >> 4;
  const size_t wrow_bytes = size_t(36) * (K / 64);

  // A staging: thread -> tile row ar = tid >> 1, chunks 4 ac .. 4 ac + 3 (64 contiguous bytes of the step).
  // Rows past the tile's end read the tile's first row instead (their results are never stored).
  const int ar = tid >> 1, ac = tid & 1;
  const u32x4 *a_ptr;
  {
    const int p = row0 + (ar < rows ? ar : 0);
    const size_t r = MODE == MODE_GATE_UP ? size_t(order[p] / uint32_t(topk)) : size_t(p);
    a_ptr = reinterpret_cast<const u32x4 *>(a_src + r * K + 32 * ac);
  }
  // weight staging: thread -> tile feature tid
  const uint8_t *w_row;
  if (MODE == MODE_GATE_UP)
    w_row = (tid < GN / 2 ? w0 : w1) + (size_t(e) * n_rows + nt * (GN / 2) + (tid % (GN / 2))) * wrow_bytes;
  else
    w_row = w0 + (size_t(e) * n_rows + nt * GN + tid) * wrow_bytes;

  // tile features of this wave's 4 fragments: gate/up: gate 32 w + 16 nb (nb < 2), up 128 + 32 w + 16 (nb - 2)
  // (the same features); down: 64 w + 16 nb
  int fbase[4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
    fbase[nb] = MODE == MODE_GATE_UP ? (nb < 2 ? 32 * wave + 16 * nb : GN / 2 + 32 * wave + 16 * (nb - 2))
                                     : 64 * wave + 16 * nb;

  u32x4 areg[4];
  uint32_t wraw[RawW<TB>::N];
  f32x4 acc[4][8];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) acc[nb][mb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  auto load = [&](int kk) {  // raw weights and A of step kk into registers
    load_w<TB>(w_row, kk, wraw);
#pragma unroll
    for (int i = 0; i < 4; ++i) areg[i] = a_ptr[size_t(kk) * (GK / 8) + i];
  };
  auto stage = [&](int l, int kk) {  // registers -> LDS stage l
#pragma unroll
    for (int j = 0; j < 4; ++j) As[l][achunk(ar, 4 * ac + j)] = areg[j];
    uint32_t o[kWp];
    pack_w<TB>(wraw, kk, o);
#pragma unroll
    for (int j = 0; j < kWp; ++j) Wp[l][tid * kWp + j] = o[j];
  };
  // 64 MFMAs out of LDS stage l: per K slice, the 4 weight fragments are decoded from their packed words, then
  // each A fragment meets all 4
  auto compute = [&](int l) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      half8 wf[4];
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        const int f = fbase[nb] + fr;
        wf[nb] = decode8<TB>(Wp[l][f * kWp + 4 * ks + g], Wp[l][f * kWp + 8 + (TB == LMOE_Q4_K ? ks : 0)], ks);
      }
#pragma unroll
      for (int mb = 0; mb < 8; ++mb) {
        const half8 xf = __builtin_bit_cast(half8, As[l][achunk(16 * mb + fr, 4 * ks + g)]);
#pragma unroll
        for (int nb = 0; nb < 4; ++nb)
          acc[nb][mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[nb], xf, acc[nb][mb], 0, 0, 0);
      }
    }
  };
  // Step kk: issue the global loads of step kk + 1, multiply out of LDS stage kk % 2 (the loads are in flight
  // meanwhile), then repack step kk + 1 into the other stage; one barrier a step.
  const int nk = K / GK;
  load(0);
  stage(0, 0);
  __syncthreads();
  for (int kk = 0; kk + 1 < nk; ++kk) {
    load(kk + 1);
    __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of the MFMAs (the scheduler sinks them otherwise)
    compute(kk & 1);
    stage((kk + 1) & 1, kk + 1);
    __syncthreads();
  }
  compute((nk - 1) & 1);

  // acc[nb][mb][r] = D[tile feature fbase[nb] + 4 g + r][token row 16 mb + fr]
#pragma unroll
  for (int mb = 0; mb < 8; ++mb) {
    const int m = 16 * mb + fr;
    if (m >= rows) continue;
    const size_t o = size_t(row0 + m) * ldo;
    if (MODE == MODE_GATE_UP) {
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        h2_t v01 = {_Float16(silu_mul(acc[nb][mb][0], acc[nb + 2][mb][0])),
                    _Float16(silu_mul(acc[nb][mb][1], acc[nb + 2][mb][1]))};
        h2_t v23 = {_Float16(silu_mul(acc[nb][mb][2], acc[nb + 2][mb][2])),
                    _Float16(silu_mul(acc[nb][mb][3], acc[nb + 2][mb][3]))};
        *reinterpret_cast<u32x2 *>(static_cast<_Float16 *>(out) + o + nt * (GN / 2) + fbase[nb] + 4 * g) =
            u32x2{__builtin_bit_cast(uint32_t, v01), __builtin_bit_cast(uint32_t, v23)};
      }
    } else if (odt == LMOE_F32) {
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
        *reinterpret_cast<f32x4 *>(static_cast<float *>(out) + o + nt * GN + fbase[nb] + 4 * g) = acc[nb][mb];
    } else {
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        h2_t v01 = {_Float16(acc[nb][mb][0]), _Float16(acc[nb][mb][1])};
        h2_t v23 = {_Float16(acc[nb][mb][2]), _Float16(acc[nb][mb][3])};
        *reinterpret_cast<u32x2 *>(static_cast<_Float16 *>(out) + o + nt * GN + fbase[nb] + 4 * g) =
            u32x2{__builtin_bit_cast(uint32_t, v01), __builtin_bit_cast(uint32_t, v23)};
      }
    }
  }
}

// x [n] in dt -> f16 (round to nearest even), 8 elements a thread (vector loads when the whole range allows)
__global__ void __launch_bounds__(256) k_to_f16(const void *x, int dt, long long n, _Float16 *out, int vec) {
  const long long i0 = (static_cast<long long>(blockIdx.x) * 256 + threadIdx.x) * 8;
  if (i0 >= n) return;
  if (vec) {
    float v[8];
    load8(x, size_t(i0), dt, v);
    store8(out, size_t(i0), LMOE_F16, v);
    return;
  }
  const int cnt = int(min(8ll, n - i0));
#pragma unroll
  for (int i = 0; i < 8; ++i)
    if (i < cnt) out[i0 + i] = _Float16(load_elt(x, size_t(i0 + i), dt));
}

}  // namespace lmoe

using namespace lmoe;

extern "C" int lmoe_grouped_tile_rows(void) { return GM; }

extern "C" int lmoe_to_f16(const void *x, int xdtype, long long n, void *out, void *stream) {
  const char *fn = "lmoe_to_f16";
  LMOE_REQUIRE(dtype_ok(xdtype), LMOE_EINVAL, "%s: bad dtype", fn);
  LMOE_REQUIRE(n >= 0, LMOE_ESHAPE, "%s: negative length", fn);
  if (n == 0) return 0;
  LMOE_REQUIRE(x && out, LMOE_EINVAL, "%s: null pointer", fn);
  const long long blocks = (n + 2047) / 2048;
  LMOE_REQUIRE(blocks < (1ll << 31), LMOE_ESHAPE, "%s: %lld elements", fn, n);
  const int vec = n % 8 == 0 && aligned16(x) && aligned16(out);
  launch(k_to_f16, dim3(unsigned(blocks)), dim3(256), 0, (hipStream_t)stream, x, xdtype, n,
         static_cast<_Float16 *>(out), vec);
  LMOE_LAUNCHED(fn);
  return 0;
}

extern "C" int lmoe_grouped_gate_up(const void *x, int xdtype, int T, int topk, const uint32_t *order,
                                    const uint32_t *offsets, const uint32_t *tiles, const uint32_t *n_tiles,
                                    int max_tiles, const uint8_t *wg, const uint8_t *wu, int type_g, int type_u,
                                    int n_experts, int H, int I, void *h, void *stream) {
  const char *fn = "lmoe_grouped_gate_up";
  LMOE_REQUIRE(qtype_ok(type_g) && qtype_ok(type_u), LMOE_ETYPE,
               "%s: ggml types %d/%d are not supported (Q4_0 = 2, Q4_K = 12)", fn, type_g, type_u);
  LMOE_REQUIRE(type_g == type_u, LMOE_ETYPE, "%s: gate and up must share one type on this path (%d vs %d)", fn,
               type_g, type_u);
  LMOE_REQUIRE(xdtype == LMOE_F16, LMOE_EINVAL,
               "%s: x must be float16 here (convert once with lmoe_to_f16; the matrix cores read f16)", fn);
  LMOE_REQUIRE(T >= 0 && topk > 0 && n_experts > 0 && max_tiles >= 0, LMOE_ESHAPE, "%s: bad shape", fn);
  LMOE_REQUIRE(H > 0 && H % block_weights(type_g) == 0 && H % 64 == 0, LMOE_ESHAPE,
               "%s: hidden size %d is not a multiple of %d", fn, H, type_g == LMOE_Q4_K ? 256 : 64);
  LMOE_REQUIRE(I > 0 && I % (GN / 2) == 0, LMOE_ESHAPE, "%s: intermediate size %d is not a multiple of %d", fn, I,
               GN / 2);
  if (T == 0 || max_tiles == 0) return 0;
  LMOE_REQUIRE(x && order && offsets && tiles && n_tiles && wg && wu && h, LMOE_EINVAL, "%s: null pointer", fn);
  LMOE_REQUIRE(aligned16(x) && aligned16(h) && aligned4(wg) && aligned4(wu), LMOE_EALIGN,
               "%s: x and h must be 16-byte aligned, weights 4-byte aligned", fn);
  const int n_ntile = I / (GN / 2);
  const long long grid = (long long)n_ntile * max_tiles;
  LMOE_REQUIRE(grid < (1ll << 31), LMOE_ESHAPE, "%s: %lld workgroups", fn, grid);
  hipStream_t st = (hipStream_t)stream;
  const _Float16 *a = static_cast<const _Float16 *>(x);
  if (type_g == LMOE_Q4_0)
    launch(k_grouped<MODE_GATE_UP, LMOE_Q4_0>, dim3(unsigned(grid)), dim3(kThreads), 0, st, a, topk, order, offsets,
           tiles, n_tiles, n_ntile, wg, wu, H, I, h, I, int(LMOE_F16));
  else
    launch(k_grouped<MODE_GATE_UP, LMOE_Q4_K>, dim3(unsigned(grid)), dim3(kThreads), 0, st, a, topk, order, offsets,
           tiles, n_tiles, n_ntile, wg, wu, H, I, h, I, int(LMOE_F16));
  LMOE_LAUNCHED(fn);
  return 0;
}

extern "C" int lmoe_grouped_down(const void *h, const uint32_t *offsets, const uint32_t *tiles,
                                 const uint32_t *n_tiles, int max_tiles, const uint8_t *wd, int type_d, int n_experts,
                                 int I, int H, void *y, int ydtype, void *stream) {
  const char *fn = "lmoe_grouped_down";
  LMOE_REQUIRE(qtype_ok(type_d), LMOE_ETYPE, "%s: ggml type %d is not supported (Q4_0 = 2, Q4_K = 12)", fn, type_d);
  LMOE_REQUIRE(n_experts > 0 && max_tiles >= 0, LMOE_ESHAPE, "%s: bad shape", fn);
  LMOE_REQUIRE(I > 0 && I % block_weights(type_d) == 0 && I % 64 == 0, LMOE_ESHAPE,
               "%s: intermediate size %d is not a multiple of %d", fn, I, type_d == LMOE_Q4_K ? 256 : 64);
  LMOE_REQUIRE(H > 0 && H % GN == 0, LMOE_ESHAPE, "%s: hidden size %d is not a multiple of %d", fn, H, GN);
  LMOE_REQUIRE(ydtype == LMOE_F16 || ydtype == LMOE_F32, LMOE_EINVAL, "%s: y must be float16 or float32", fn);
  if (max_tiles == 0) return 0;
  LMOE_REQUIRE(h && offsets && tiles && n_tiles && wd && y, LMOE_EINVAL, "%s: null pointer", fn);
  LMOE_REQUIRE(aligned16(h) && aligned16(y) && aligned4(wd), LMOE_EALIGN,
               "%s: h and y must be 16-byte aligned, weights 4-byte aligned", fn);
  const int n_ntile = H / GN;
  const long long grid = (long long)n_ntile * max_tiles;
  LMOE_REQUIRE(grid < (1ll << 31), LMOE_ESHAPE, "%s: %lld workgroups", fn, grid);
  hipStream_t st = (hipStream_t)stream;
  const _Float16 *a = static_cast<const _Float16 *>(h);
  if (type_d == LMOE_Q4_0)
    launch(k_grouped<MODE_DOWN, LMOE_Q4_0>, dim3(unsigned(grid)), dim3(kThreads), 0, st, a, 1,
           static_cast<const uint32_t *>(nullptr), offsets, tiles, n_tiles, n_ntile, wd,
           static_cast<const uint8_t *>(nullptr), I, H, y, H, ydtype);
  else
    launch(k_grouped<MODE_DOWN, LMOE_Q4_K>, dim3(unsigned(grid)), dim3(kThreads), 0, st, a, 1,
           static_cast<const uint32_t *>(nullptr), offsets, tiles, n_tiles, n_ntile, wd,
           static_cast<const uint8_t *>(nullptr), I, H, y, H, ydtype);
  LMOE_LAUNCHED(fn);
  return 0;
}
