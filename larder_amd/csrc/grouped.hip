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
//   * each K step of 64 stages an A tile of 128 rows (gate/up: rows of x gathered through the grouped order and
//     converted to f16; down: the grouped h rows) and a W tile of 128 weight rows decoded from Q4_0 / Q4_K to f16
//     ((q - 8) d, d sc q - dmin m) into LDS, double-buffered: the next step's global loads are in flight while the
//     current step's MFMAs run;
//   * four wavefronts each own a 64 x 64 corner (4 x 4 accumulators of 16 x 16). The weights are the MFMA's first
//     operand, so each lane ends with 4 consecutive output features of one row and stores 8 bytes;
//   * gate/up tiles hold 64 gate and 64 up rows of the same intermediate features: SwiGLU happens in registers and
//     h leaves as f16 in grouped row order. Down writes y [R][H] f16 in grouped order for lmoe_combine_sorted.
// Operands are f16 with fp32 accumulation. A single rounding of (q - 8) d to f16 keeps the layer well inside the
// 2e-3 relative L2 bar; bf16 operands would not.
#include "lmoe_common.h"

namespace lmoe {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int GM = 128;       // rows a tile (the grouping kernel's bm)
constexpr int GN = 128;       // output columns a tile (gate/up: 64 gate + 64 up features)
constexpr int GK = 64;        // K a step
constexpr int LDA = GK + 8;   // halves a staged row: the 16-byte pad spreads 16-byte lane reads over all banks
constexpr int kTileMask = (1 << 20) - 1;

enum { MODE_GATE_UP = 0, MODE_DOWN = 1 };

// four f16 (1024 + q) from the low nibbles of a byte-wise masked word: {q0, q1} and {q2, q3}
__device__ __forceinline__ uint32_t magic_pair(uint32_t nib, uint32_t sel) {
  return __builtin_amdgcn_perm(0x64646464u, nib, sel);
}
constexpr uint32_t kSel01 = 0x04010400u, kSel23 = 0x04030402u;

// 8 f16 weights (one lane's LDS quadword) from the 4 nibbles of `nib` (already masked to one nibble a byte):
// values (1024 + q - bias) * scale - sub, written as pairs in natural order
__device__ __forceinline__ void decode4(uint32_t nib, h2_t bias, h2_t scale, h2_t sub, uint32_t *o) {
  const h2_t a = __builtin_bit_cast(h2_t, magic_pair(nib, kSel01));
  const h2_t b = __builtin_bit_cast(h2_t, magic_pair(nib, kSel23));
  o[0] = __builtin_bit_cast(uint32_t, (a - bias) * scale - sub);
  o[1] = __builtin_bit_cast(uint32_t, (b - bias) * scale - sub);
}

// Q4_0 block (f16 d, 16 qs words) -> 32 f16 (q - 8) d in natural order, as 16 words
__device__ __forceinline__ void dequant_q4_0_block(const uint32_t qs[4], float d, uint32_t o[16]) {
  const _Float16 dh = _Float16(d);
  const h2_t bias = {_Float16(1032.0f), _Float16(1032.0f)}, scale = {dh, dh}, zero = {_Float16(0.0f), _Float16(0.0f)};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    decode4(qs[i] & 0x0F0F0F0Fu, bias, scale, zero, o + 2 * i);             // elements 4i .. 4i + 3
    decode4((qs[i] >> 4) & 0x0F0F0F0Fu, bias, scale, zero, o + 8 + 2 * i);  // elements 16 + 4i ..
  }
}

// Q4_K: 16 consecutive qs bytes of one sub-block pair -> 16 f16 of sub-block lo (low nibbles, scale d1 / min m1)
// and 16 of sub-block hi (high nibbles, d2 / m2): d sc q - dmin m, scale and min rounded to f16 first
__device__ __forceinline__ void dequant_q4_k_half(const uint32_t qs[4], float d1, float m1, float d2, float m2,
                                                  uint32_t lo[8], uint32_t hi[8]) {
  const h2_t bias = {_Float16(1024.0f), _Float16(1024.0f)};
  const h2_t s1 = {_Float16(d1), _Float16(d1)}, n1 = {_Float16(m1), _Float16(m1)};
  const h2_t s2 = {_Float16(d2), _Float16(d2)}, n2 = {_Float16(m2), _Float16(m2)};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    decode4(qs[i] & 0x0F0F0F0Fu, bias, s1, n1, lo + 2 * i);
    decode4((qs[i] >> 4) & 0x0F0F0F0Fu, bias, s2, n2, hi + 2 * i);
  }
}

// x elements -> f16 pairs
template <int ADT>
__device__ __forceinline__ uint32_t to_f16_pair(uint32_t a, uint32_t b) {
  if (ADT == LMOE_BF16) {  // bf16 pair in one word; exact in f16 over f16's normal range
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(__uint_as_float(a << 16),
                                                                 __uint_as_float(a & 0xFFFF0000u)));
  } else {  // two f32 words, rounded to nearest
    const h2_t v = {_Float16(__uint_as_float(a)), _Float16(__uint_as_float(b))};
    return __builtin_bit_cast(uint32_t, v);
  }
}

// Grid: n_ntile * max_tiles workgroups of 256 threads (1-D). GATE_UP: n-tile j covers intermediate features
// 64 j .. 64 j + 63 (gate rows in W rows 0..63 of the tile, up rows in 64..127), K = H, A rows x[order[p] / topk],
// out h [R][I] f16. DOWN: n-tile j covers output features 128 j .., K = I, A rows h[p], out y [R][H] f16.
template <int MODE, int TB, int ADT>
__global__ void __launch_bounds__(256, 2)
    k_grouped(const void *a_src, int topk, const uint32_t *order, const uint32_t *offsets, const uint32_t *tiles,
              const uint32_t *n_tiles, int n_ntile, const uint8_t *w0, const uint8_t *w1, int K, int n_rows,
              void *out, int ldo, int odt) {
  __shared__ __attribute__((aligned(16))) _Float16 As[2][GM * LDA];
  __shared__ __attribute__((aligned(16))) _Float16 Ws[2][GN * LDA];

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
  const int P = K / 64;  // 64-weight units a weight row
  const size_t wrow_bytes = size_t(36) * P;

  // A staging: thread -> row am of the tile, 32 elements from k offset ak of each step
  constexpr int AES = ADT == LMOE_F32 ? 4 : 2;  // bytes an element
  constexpr int AV = 32 * AES / 16;              // 16-byte loads a step
  const int am = tid >> 1, ak = (tid & 1) * 32;
  const bool a_ok = am < rows;
  const u32x4 *a_ptr = nullptr;
  if (a_ok) {
    const int p = row0 + am;
    const size_t r = MODE == MODE_GATE_UP ? size_t(order[p] / uint32_t(topk)) : size_t(p);
    a_ptr = reinterpret_cast<const u32x4 *>(static_cast<const char *>(a_src) + (r * K + ak) * AES);
  }
  // W staging: thread -> weight row wn of the tile, part wp (Q4_0: block wp of the unit; Q4_K: qs bytes 16 wp ..)
  const int wn = tid >> 1, wp = tid & 1;
  const uint8_t *w_row;
  if (MODE == MODE_GATE_UP)
    w_row = (wn < 64 ? w0 : w1) + (size_t(e) * n_rows + nt * 64 + (wn & 63)) * wrow_bytes;
  else
    w_row = w0 + (size_t(e) * n_rows + nt * GN + wn) * wrow_bytes;

  u32x4 areg[AV];
  uint32_t wreg[TB == LMOE_Q4_0 ? 5 : 8];
  auto load = [&](int kk) {
    if (a_ok) {
#pragma unroll
      for (int i = 0; i < AV; ++i) areg[i] = a_ptr[size_t(kk) * (GK * AES / 16) + i];
    }
    if (TB == LMOE_Q4_0) {  // block wp of unit kk: words 4 wp .. 4 wp + 4 of the 36-byte unit
      const uint32_t *u = reinterpret_cast<const uint32_t *>(w_row + size_t(kk) * 36) + 4 * wp;
#pragma unroll
      for (int i = 0; i < 5; ++i) wreg[i] = u[i];
    } else {  // superblock kk / 4, sub-block pair kk % 4: header words 0..3, qs words 4 + 8 (kk % 4) + 4 wp ..
      const uint32_t *sb = reinterpret_cast<const uint32_t *>(w_row + size_t(kk >> 2) * 144);
#pragma unroll
      for (int i = 0; i < 4; ++i) wreg[i] = sb[i];
#pragma unroll
      for (int i = 0; i < 4; ++i) wreg[4 + i] = sb[4 + 8 * (kk & 3) + 4 * wp + i];
    }
  };
  auto store = [&](int buf, int kk) {
    if (a_ok) {
      u32x4 *ad = reinterpret_cast<u32x4 *>(&As[buf][am * LDA + ak]);
      if (ADT == LMOE_F16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) ad[i] = areg[i];
      } else if (ADT == LMOE_BF16) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          ad[i] = u32x4{to_f16_pair<ADT>(areg[i].x, 0), to_f16_pair<ADT>(areg[i].y, 0),
                        to_f16_pair<ADT>(areg[i].z, 0), to_f16_pair<ADT>(areg[i].w, 0)};
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          ad[i] = u32x4{to_f16_pair<ADT>(areg[2 * i].x, areg[2 * i].y), to_f16_pair<ADT>(areg[2 * i].z, areg[2 * i].w),
                        to_f16_pair<ADT>(areg[2 * i + 1].x, areg[2 * i + 1].y),
                        to_f16_pair<ADT>(areg[2 * i + 1].z, areg[2 * i + 1].w)};
      }
    }
    if (TB == LMOE_Q4_0) {
      uint32_t qs[4], o[16];
      float d;
      if (wp == 0) {  // block 0 starts at byte 0: d in the low half of word 0, qs at bytes 2..17
        d = half_lo(wreg[0]);
#pragma unroll
        for (int i = 0; i < 4; ++i) qs[i] = __builtin_amdgcn_alignbyte(wreg[i + 1], wreg[i], 2);
      } else {  // block 1 starts at byte 18: d in the high half of word 4, qs in words 5..8
        d = half_hi(wreg[0]);
#pragma unroll
        for (int i = 0; i < 4; ++i) qs[i] = wreg[i + 1];
      }
      dequant_q4_0_block(qs, d, o);
      u32x4 *wd = reinterpret_cast<u32x4 *>(&Ws[buf][wn * LDA + 32 * wp]);
#pragma unroll
      for (int i = 0; i < 4; ++i) wd[i] = u32x4{o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]};
    } else {
      const int c = kk & 3;
      float sc1, mn1, sc2, mn2;
      k4_scale_min(wreg[1], wreg[2], wreg[3], 2 * c, &sc1, &mn1);
      k4_scale_min(wreg[1], wreg[2], wreg[3], 2 * c + 1, &sc2, &mn2);
      const float d = half_lo(wreg[0]), dmin = half_hi(wreg[0]);
      uint32_t lo[8], hi[8];
      dequant_q4_k_half(wreg + 4, d * sc1, dmin * mn1, d * sc2, dmin * mn2, lo, hi);
      u32x4 *wl = reinterpret_cast<u32x4 *>(&Ws[buf][wn * LDA + 16 * wp]);       // k = 16 wp + j
      u32x4 *wh = reinterpret_cast<u32x4 *>(&Ws[buf][wn * LDA + 32 + 16 * wp]);  // k = 32 + 16 wp + j
      wl[0] = u32x4{lo[0], lo[1], lo[2], lo[3]};
      wl[1] = u32x4{lo[4], lo[5], lo[6], lo[7]};
      wh[0] = u32x4{hi[0], hi[1], hi[2], hi[3]};
      wh[1] = u32x4{hi[4], hi[5], hi[6], hi[7]};
    }
  };

  // wavefront corner: token rows 64 wm .. (A rows of the tile), weight rows per jn (gate/up: 32 gate rows
  // 32 wv .. and the 32 up rows 64 + 32 wv .. of the same features; down: 64 wv ..)
  const int wm = wave >> 1, wv = wave & 1;
  int wbase[4];
#pragma unroll
  for (int jn = 0; jn < 4; ++jn)
    wbase[jn] = MODE == MODE_GATE_UP ? (jn < 2 ? 32 * wv + 16 * jn : 64 + 32 * wv + 16 * (jn - 2)) : 64 * wv + 16 * jn;
  const int fr = lane & 15, fk = (lane >> 4) * 8;

  f32x4 acc[4][4];
#pragma unroll
  for (int jn = 0; jn < 4; ++jn)
#pragma unroll
    for (int im = 0; im < 4; ++im) acc[jn][im] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  const int nk = K / GK;
  load(0);
  store(0, 0);
  __syncthreads();
  for (int kk = 0; kk < nk; ++kk) {
    const int cur = kk & 1;
    if (kk + 1 < nk) load(kk + 1);
#pragma unroll
    for (int ks = 0; ks < GK; ks += 32) {
      half8 wf[4], xf[4];
#pragma unroll
      for (int jn = 0; jn < 4; ++jn)
        wf[jn] = *reinterpret_cast<const half8 *>(&Ws[cur][(wbase[jn] + fr) * LDA + ks + fk]);
#pragma unroll
      for (int im = 0; im < 4; ++im)
        xf[im] = *reinterpret_cast<const half8 *>(&As[cur][(64 * wm + 16 * im + fr) * LDA + ks + fk]);
#pragma unroll
      for (int jn = 0; jn < 4; ++jn)
#pragma unroll
        for (int im = 0; im < 4; ++im)
          acc[jn][im] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[jn], xf[im], acc[jn][im], 0, 0, 0);
    }
    if (kk + 1 < nk) store(cur ^ 1, kk + 1);
    __syncthreads();
  }

  // acc[jn][im][r] = D[weight row wbase[jn] + 4 (lane / 16) + r][token row 64 wm + 16 im + lane % 16]
  const int orow = 4 * (lane >> 4);
#pragma unroll
  for (int im = 0; im < 4; ++im) {
    const int m = 64 * wm + 16 * im + fr;
    if (m >= rows) continue;
    const size_t o = size_t(row0 + m) * ldo;
    if (MODE == MODE_GATE_UP) {
#pragma unroll
      for (int jn = 0; jn < 2; ++jn) {
        h2_t v01 = {_Float16(silu_mul(acc[jn][im][0], acc[jn + 2][im][0])),
                    _Float16(silu_mul(acc[jn][im][1], acc[jn + 2][im][1]))};
        h2_t v23 = {_Float16(silu_mul(acc[jn][im][2], acc[jn + 2][im][2])),
                    _Float16(silu_mul(acc[jn][im][3], acc[jn + 2][im][3]))};
        *reinterpret_cast<u32x2 *>(static_cast<_Float16 *>(out) + o + nt * 64 + wbase[jn] + orow) =
            u32x2{__builtin_bit_cast(uint32_t, v01), __builtin_bit_cast(uint32_t, v23)};
      }
    } else if (odt == LMOE_F32) {
#pragma unroll
      for (int jn = 0; jn < 4; ++jn)
        *reinterpret_cast<f32x4 *>(static_cast<float *>(out) + o + nt * GN + wbase[jn] + orow) = acc[jn][im];
    } else {
#pragma unroll
      for (int jn = 0; jn < 4; ++jn) {
        h2_t v01 = {_Float16(acc[jn][im][0]), _Float16(acc[jn][im][1])};
        h2_t v23 = {_Float16(acc[jn][im][2]), _Float16(acc[jn][im][3])};
        *reinterpret_cast<u32x2 *>(static_cast<_Float16 *>(out) + o + nt * GN + wbase[jn] + orow) =
            u32x2{__builtin_bit_cast(uint32_t, v01), __builtin_bit_cast(uint32_t, v23)};
      }
    }
  }
}

template <int MODE, int TB>
static void grouped_launch(int adt, int grid, hipStream_t st, const void *a, int topk, const uint32_t *order,
                           const uint32_t *offsets, const uint32_t *tiles, const uint32_t *n_tiles, int n_ntile,
                           const uint8_t *w0, const uint8_t *w1, int K, int n_rows, void *out, int ldo, int odt) {
  if (MODE == MODE_DOWN || adt == LMOE_F16)
    launch(k_grouped<MODE, TB, LMOE_F16>, dim3(grid), dim3(256), 0, st, a, topk, order, offsets, tiles, n_tiles,
           n_ntile, w0, w1, K, n_rows, out, ldo, odt);
  else if constexpr (MODE == MODE_GATE_UP) {
    if (adt == LMOE_BF16)
      launch(k_grouped<MODE, TB, LMOE_BF16>, dim3(grid), dim3(256), 0, st, a, topk, order, offsets, tiles, n_tiles,
           n_ntile, w0, w1, K, n_rows, out, ldo, odt);
    else
      launch(k_grouped<MODE, TB, LMOE_F32>, dim3(grid), dim3(256), 0, st, a, topk, order, offsets, tiles, n_tiles,
             n_ntile, w0, w1, K, n_rows, out, ldo, odt);
  }
}

}  // namespace lmoe

using namespace lmoe;

extern "C" int lmoe_grouped_tile_rows(void) { return GM; }

extern "C" int lmoe_grouped_gate_up(const void *x, int xdtype, int T, int topk, const uint32_t *order,
                                    const uint32_t *offsets, const uint32_t *tiles, const uint32_t *n_tiles,
                                    int max_tiles, const uint8_t *wg, const uint8_t *wu, int type_g, int type_u,
                                    int n_experts, int H, int I, void *h, void *stream) {
  const char *fn = "lmoe_grouped_gate_up";
  LMOE_REQUIRE(qtype_ok(type_g) && qtype_ok(type_u), LMOE_ETYPE,
               "%s: ggml types %d/%d are not supported (Q4_0 = 2, Q4_K = 12)", fn, type_g, type_u);
  LMOE_REQUIRE(type_g == type_u, LMOE_ETYPE, "%s: gate and up must share one type on this path (%d vs %d)", fn,
               type_g, type_u);
  LMOE_REQUIRE(dtype_ok(xdtype), LMOE_EINVAL, "%s: bad x dtype", fn);
  LMOE_REQUIRE(T >= 0 && topk > 0 && n_experts > 0 && max_tiles >= 0, LMOE_ESHAPE, "%s: bad shape", fn);
  LMOE_REQUIRE(H > 0 && H % block_weights(type_g) == 0 && H % 64 == 0, LMOE_ESHAPE,
               "%s: hidden size %d is not a multiple of %d", fn, H, type_g == LMOE_Q4_K ? 256 : 64);
  LMOE_REQUIRE(I > 0 && I % 64 == 0, LMOE_ESHAPE, "%s: intermediate size %d is not a multiple of 64", fn, I);
  if (T == 0 || max_tiles == 0) return 0;
  LMOE_REQUIRE(x && order && offsets && tiles && n_tiles && wg && wu && h, LMOE_EINVAL, "%s: null pointer", fn);
  LMOE_REQUIRE(aligned16(x) && aligned16(h) && aligned4(wg) && aligned4(wu), LMOE_EALIGN,
               "%s: x and h must be 16-byte aligned, weights 4-byte aligned", fn);
  const int n_ntile = I / 64;
  const long long grid = (long long)n_ntile * max_tiles;
  LMOE_REQUIRE(grid < (1ll << 31), LMOE_ESHAPE, "%s: %lld workgroups", fn, grid);
  hipStream_t st = (hipStream_t)stream;
  if (type_g == LMOE_Q4_0)
    grouped_launch<MODE_GATE_UP, LMOE_Q4_0>(xdtype, int(grid), st, x, topk, order, offsets, tiles, n_tiles, n_ntile,
                                            wg, wu, H, I, h, I, LMOE_F16);
  else
    grouped_launch<MODE_GATE_UP, LMOE_Q4_K>(xdtype, int(grid), st, x, topk, order, offsets, tiles, n_tiles, n_ntile,
                                            wg, wu, H, I, h, I, LMOE_F16);
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
  if (type_d == LMOE_Q4_0)
    grouped_launch<MODE_DOWN, LMOE_Q4_0>(LMOE_F16, int(grid), st, h, 1, nullptr, offsets, tiles, n_tiles, n_ntile, wd,
                                         nullptr, I, H, y, H, ydtype);
  else
    grouped_launch<MODE_DOWN, LMOE_Q4_K>(LMOE_F16, int(grid), st, h, 1, nullptr, offsets, tiles, n_tiles, n_ntile, wd,
                                         nullptr, I, H, y, H, ydtype);
  LMOE_LAUNCHED(fn);
  return 0;
}
