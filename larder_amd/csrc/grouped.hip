// Grouped expert GEMMs on the matrix cores, for prefill and batched decode: rows grouped by expert on the device
// (lmoe_group_rows), then one 128 x 128 output tile per (expert, m-tile, n-tile) through v_mfma_f32_16x16x32_f16.
//
// The reference's prefill path ("dense", gguf_experts.py:698-722) dequantizes up to 8 experts at a time to f16 in
// HBM (DEQ_SRC, :529-539) and runs MLX gather_mm on host-sorted rows. Here no weight is dequantized to HBM and the
// host never waits:
//   * the work list (expert << 20 | m-tile) and its length come from the grouping kernel; the 1-D grid is sized
//     for the most tiles R rows can make and workgroups past the device-side count exit at once. Workgroups are
//     dealt round-robin over the 8 XCDs, so the linear id is remapped to give each XCD one contiguous stretch of
//     work (neighbouring n-tiles of one m-tile share A rows and the expert's weights in that XCD's L2);
//   * each K step of 64 stages an A tile of 128 rows (gate/up: rows of x, already f16, gathered through the
//     grouped order; down: the grouped h rows) and a W tile of 128 weight rows decoded from Q4_0 / Q4_K to f16
//     ((q - 8) d, d sc q - dmin m) into LDS, double-buffered, 16-byte chunks XOR-swizzled by row so that both the
//     staging writes and the MFMA fragment reads are free of bank conflicts. Each thread moves 64 contiguous bytes
//     of one A row a step, so the row gather costs few address transactions; global loads run two steps ahead
//     of the MFMAs that use them;
//   * four wavefronts each own a 64 x 64 corner (4 x 4 accumulators of 16 x 16, in VGPRs; two workgroups a CU,
//     so two waves share each SIMD and cover each other's waits). The weights are the MFMA's first operand, so
//     each lane ends with 4 consecutive output features of one row;
//   * gate/up tiles hold 64 gate and 64 up rows of the same intermediate features: SwiGLU happens in registers
//     and h leaves as f16 in grouped row order. Down writes y [R][H] (f16 or f32) in grouped order.
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
constexpr int GK = 64;   // K a step
constexpr int kThreads = 512;
constexpr int kTileMask = (1 << 20) - 1;

enum { MODE_GATE_UP = 0, MODE_DOWN = 1 };

template <int N>
using IC = std::integral_constant<int, N>;

// 16-byte chunk c (0..7) of W row r in a stage: rows are 128 bytes, chunks XOR-swizzled by the row's low 3 bits
__device__ __forceinline__ int wchunk(int r, int c) { return r * 8 + (c ^ (r & 7)); }

// four f16 (1024 + q) from a byte-wise masked word: {q0, q1} and {q2, q3}
__device__ __forceinline__ uint32_t magic_pair(uint32_t nib, uint32_t sel) {
  return __builtin_amdgcn_perm(0x64646464u, nib, sel);
}
constexpr uint32_t kSel01 = 0x04010400u, kSel23 = 0x04030402u;

// 4 f16 weights from the 4 nibbles of `nib` (one nibble a byte): ((1024 + q) - bias) * scale - sub, as 2 pairs
__device__ __forceinline__ void decode4(uint32_t nib, h2_t bias, h2_t scale, h2_t sub, uint32_t *o) {
  const h2_t a = __builtin_bit_cast(h2_t, magic_pair(nib, kSel01));
  const h2_t b = __builtin_bit_cast(h2_t, magic_pair(nib, kSel23));
  o[0] = __builtin_bit_cast(uint32_t, (a - bias) * scale - sub);
  o[1] = __builtin_bit_cast(uint32_t, (b - bias) * scale - sub);
}

// Raw words a thread loads for one (weight row, part) of a K step
template <int TB>
struct Raw {
  static constexpr int N = TB == LMOE_Q4_0 ? 5 : 12;
};

// Load the raw words of (row `wrow`, part h) for K step kk. Q4_0: block h of unit kk is words 4h .. 4h + 4 of
// the 36-byte unit. Q4_K: super-block kk / 4 header words 0..3 and the 8 qs words of sub-block pair kk % 4.
template <int TB>
__device__ __forceinline__ void load_raw(const uint8_t *wrow, int h, int kk, uint32_t *r) {
  if (TB == LMOE_Q4_0) {
    const uint32_t *u = reinterpret_cast<const uint32_t *>(wrow + size_t(kk) * 36) + 4 * h;
#pragma unroll
    for (int i = 0; i < 5; ++i) r[i] = u[i];
  } else {
    const uint32_t *sb = reinterpret_cast<const uint32_t *>(wrow + size_t(kk >> 2) * 144);
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = sb[i];
#pragma unroll
    for (int i = 0; i < 8; ++i) r[4 + i] = sb[4 + 8 * (kk & 3) + i];
  }
}

// Decoding one (row, part h) of K step kk to 32 f16 weights = chunks 4h .. 4h + 3 of the row, one 16-byte chunk
// (8 weights) at a time so the work can sit between MFMAs. Q4_0 part h is block h: elements 0..15 from the low
// nibbles of qs bytes 0..15, 16..31 from the high ones; w = ((1024 + q) - 1032) d. Q4_K part h is sub-block
// 2 (kk % 4) + h, the low (h = 0) or high (h = 1) nibbles of the pair's 32 qs bytes; w = (q (d sc)) - dmin m.
struct Dq {
  h2_t bias, scale, sub;
};

template <int TB>
__device__ __forceinline__ Dq dq_params(const uint32_t *r, int h, int kk) {
  Dq q;
  if (TB == LMOE_Q4_0) {
    const _Float16 dh = _Float16(h == 0 ? half_lo(r[0]) : half_hi(r[0]));  // d of block 0 / block 1
    q.bias = h2_t{_Float16(1032.0f), _Float16(1032.0f)};
    q.scale = h2_t{dh, dh};
    q.sub = h2_t{_Float16(0.0f), _Float16(0.0f)};
  } else {
    float sc, mn;
    k4_scale_min(r[1], r[2], r[3], 2 * (kk & 3) + h, &sc, &mn);
    const _Float16 d1 = _Float16(half_lo(r[0]) * sc), m1 = _Float16(half_hi(r[0]) * mn);
    q.bias = h2_t{_Float16(1024.0f), _Float16(1024.0f)};
    q.scale = h2_t{d1, d1};
    q.sub = h2_t{m1, m1};
  }
  return q;
}

// chunk j (0..3) of (row, part h): weights 8 j .. 8 j + 7 of the part
template <int TB>
__device__ __forceinline__ u32x4 dq_chunk(const uint32_t *r, int h, const Dq &q, int j) {
  uint32_t w0, w1, o[4];
  int shift;
  if (TB == LMOE_Q4_0) {  // qs words (2j, 2j + 1) mod 4, low nibbles for j < 2, high for j >= 2
    const int i = 2 * (j & 1);
    if (h == 0) {  // block 0's qs start at byte 2
      w0 = __builtin_amdgcn_alignbyte(r[i + 1], r[i], 2);
      w1 = __builtin_amdgcn_alignbyte(r[i + 2], r[i + 1], 2);
    } else {  // block 1's qs are words 5..8 (r[1..4])
      w0 = r[i + 1];
      w1 = r[i + 2];
    }
    shift = j < 2 ? 0 : 4;
  } else {  // qs words 2j, 2j + 1 of the pair, nibble h
    w0 = r[4 + 2 * j];
    w1 = r[5 + 2 * j];
    shift = 4 * h;
  }
  decode4((w0 >> shift) & 0x0F0F0F0Fu, q.bias, q.scale, q.sub, o);
  decode4((w1 >> shift) & 0x0F0F0F0Fu, q.bias, q.scale, q.sub, o + 2);
  return u32x4{o[0], o[1], o[2], o[3]};
}

// Grid: n_ntile * max_tiles workgroups of 512 threads (1-D), one a CU, two waves a SIMD. GATE_UP: n-tile j
// covers intermediate features 128 j .. 128 j + 127 (W rows 0..127 of the tile are their gate rows, 128..255
// their up rows), K = H, A rows x[order[p] / topk], out h [R][I] f16. DOWN: n-tile j covers output features
// 256 j .., K = I, A rows h[p], out y [R][H] in odt (F16 / F32).
template <int MODE, int TB>
__global__ void __launch_bounds__(kThreads, 1)
k_grouped(const _Float16 *a_src, int topk, const uint32_t *order, const uint32_t *offsets, const uint32_t *tiles,
          const uint32_t *n_tiles, int n_ntile, const uint8_t *w0, const uint8_t *w1, int K, int n_rows, void *out,
          int ldo, int odt) {
  // A and W tiles, 2 stages each: rows of 64 halves = 8 chunks of 16 bytes, chunks swizzled by wchunk()
  __shared__ __attribute__((aligned(16))) u32x4 As[2][GM * 8];
  __shared__ __attribute__((aligned(16))) u32x4 Ws[2][GN * 8];

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
  const int wm = wave & 1, wn = wave >> 1;  // 2 x 4 waves of 64 x 64
  const int fr = lane & 15, g = lane >> 4;
  const size_t wrow_bytes = size_t(36) * (K / 64);

  // A staging: thread -> tile row ar = tid >> 2, chunks 2 ac, 2 ac + 1 (32 contiguous bytes of the step).
  // Rows past the tile's end read the tile's first row instead (their results are never stored).
  const int ar = tid >> 2, ac = tid & 3;
  const u32x4 *a_ptr;
  {
    const int p = row0 + (ar < rows ? ar : 0);
    const size_t r = MODE == MODE_GATE_UP ? size_t(order[p] / uint32_t(topk)) : size_t(p);
    a_ptr = reinterpret_cast<const u32x4 *>(a_src + r * K + 16 * ac);
  }
  // W staging: thread -> tile row sr = tid >> 1, part sh = tid & 1 (Q4_0 block / Q4_K sub-block sh = chunks
  // 4 sh .. 4 sh + 3)
  const int sr = tid >> 1, sh = tid & 1;
  const uint8_t *w_row;
  if (MODE == MODE_GATE_UP)
    w_row = (sr < GN / 2 ? w0 : w1) + (size_t(e) * n_rows + nt * (GN / 2) + (sr % (GN / 2))) * wrow_bytes;
  else
    w_row = w0 + (size_t(e) * n_rows + nt * GN + sr) * wrow_bytes;

  // fragment rows of W this wave reads: gate/up: gate rows 32 wn + 16 nb (nb < 2) and the up rows GN/2 + 32 wn +
  // 16 (nb - 2) of the same features; down: 64 wn + 16 nb
  int wbase[4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
    wbase[nb] =
        MODE == MODE_GATE_UP ? (nb < 2 ? 32 * wn + 16 * nb : GN / 2 + 32 * wn + 16 * (nb - 2)) : 64 * wn + 16 * nb;

  u32x4 areg[2][2];
  uint32_t wraw[2][Raw<TB>::N];
  f32x4 acc[4][4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) acc[nb][mb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  auto load = [&](auto s, int kk) {  // raw W, then A, of step kk into register stage s
    constexpr int S = decltype(s)::value;
    load_raw<TB>(w_row, sh, kk, wraw[S]);
#pragma unroll
    for (int i = 0; i < 2; ++i) areg[S][i] = a_ptr[size_t(kk) * (GK / 8) + i];
  };
  auto stage = [&](auto s, auto l, int kk) {  // register stage s -> LDS stage l
    constexpr int S = decltype(s)::value, L = decltype(l)::value;
#pragma unroll
    for (int j = 0; j < 2; ++j) As[L][wchunk(ar, 2 * ac + j)] = areg[S][j];
    const Dq q = dq_params<TB>(wraw[S], sh, kk);
#pragma unroll
    for (int j = 0; j < 4; ++j) Ws[L][wchunk(sr, 4 * sh + j)] = dq_chunk<TB>(wraw[S], sh, q, j);
  };
  const int nk = K / GK;
  // Step kk: the global loads of step kk + 2 are issued into the register stage that step kk's data left (it went
  // to LDS at the end of step kk - 1); step kk multiplies out of LDS stage kk % 2 while step kk + 1 (loaded during
  // step kk - 1) is staged into the other LDS stage, its A chunks and decoded W chunks written between groups of
  // 4 MFMAs so that a wave keeps the matrix core, the VALU and the LDS busy at once (the waves of a workgroup run
  // in lockstep between barriers, so the overlap has to come from within each wave); one barrier closes the step.
  // Past the end the step index clamps instead of branching, so the compiler's memory-counter waits stay exact.
  auto step = [&](auto sl, int kk) {
    constexpr int SL = decltype(sl)::value, SN = 1 - SL;
    load(IC<SL>{}, min(kk + 2, nk - 1));
    const int kn = min(kk + 1, nk - 1);
    const Dq q = dq_params<TB>(wraw[SN], sh, kn);
    half8 wf[2][4], xf[2][4];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
        wf[ks][nb] = __builtin_bit_cast(half8, Ws[SL][wchunk(wbase[nb] + fr, 2 * g + ks)]);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
        xf[ks][mb] = __builtin_bit_cast(half8, As[SL][wchunk(64 * wm + 16 * mb + fr, 2 * g + ks)]);
    }
#pragma unroll
    for (int grp = 0; grp < 8; ++grp) {
      const int ks = grp >> 2, mb = grp & 3;
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
        acc[nb][mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[ks][nb], xf[ks][mb], acc[nb][mb], 0, 0, 0);
      if (grp == 0) {
#pragma unroll
        for (int j = 0; j < 2; ++j) As[SN][wchunk(ar, 2 * ac + j)] = areg[SN][j];
      } else if (grp <= 4) {
        Ws[SN][wchunk(sr, 4 * sh + grp - 1)] = dq_chunk<TB>(wraw[SN], sh, q, grp - 1);
      }
    }
    __syncthreads();
  };

  load(IC<0>{}, 0);
  load(IC<1>{}, min(1, nk - 1));
  stage(IC<0>{}, IC<0>{}, 0);
  __syncthreads();
  int kk = 0;
  for (; kk + 1 < nk; kk += 2) {
    step(IC<0>{}, kk);
    step(IC<1>{}, kk + 1);
  }
  if (kk < nk) step(IC<0>{}, kk);

  // acc[nb][mb][r] = D[W row wbase[nb] + 4 g + r][token row 64 wm + 16 mb + fr]
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    const int m = 64 * wm + 16 * mb + fr;
    if (m >= rows) continue;
    const size_t o = size_t(row0 + m) * ldo;
    if (MODE == MODE_GATE_UP) {
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        h2_t v01 = {_Float16(silu_mul(acc[nb][mb][0], acc[nb + 2][mb][0])),
                    _Float16(silu_mul(acc[nb][mb][1], acc[nb + 2][mb][1]))};
        h2_t v23 = {_Float16(silu_mul(acc[nb][mb][2], acc[nb + 2][mb][2])),
                    _Float16(silu_mul(acc[nb][mb][3], acc[nb + 2][mb][3]))};
        *reinterpret_cast<u32x2 *>(static_cast<_Float16 *>(out) + o + nt * (GN / 2) + wbase[nb] + 4 * g) =
            u32x2{__builtin_bit_cast(uint32_t, v01), __builtin_bit_cast(uint32_t, v23)};
      }
    } else if (odt == LMOE_F32) {
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
        *reinterpret_cast<f32x4 *>(static_cast<float *>(out) + o + nt * GN + wbase[nb] + 4 * g) = acc[nb][mb];
    } else {
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        h2_t v01 = {_Float16(acc[nb][mb][0]), _Float16(acc[nb][mb][1])};
        h2_t v23 = {_Float16(acc[nb][mb][2]), _Float16(acc[nb][mb][3])};
        *reinterpret_cast<u32x2 *>(static_cast<_Float16 *>(out) + o + nt * GN + wbase[nb] + 4 * g) =
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
