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
//     K, f16: x gathered through the grouped order, or the grouped h rows) goes through LDS, shared by the four.
//     The weights reach LDS as raw Q4 bytes (Q4_0) or as one nibble word per (MFMA K slice, lane group) plus
//     scales (Q4_K), and each MFMA lane decodes its own 8 weights to f16 in registers, straight into the MFMA's
//     weight operand: w = ((1024 + q) - 1032) d for Q4_0, ((1024 + q) - 1024) (d sc) - dmin m for Q4_K;
//   * the K order. Inside every 32-wide block of K the GEMMs take the elements in the order
//     0-3, 16-19, 4-7, 20-23, 8-11, 24-27, 12-15, 28-31 (kperm): then MFMA lane group g's 8 weights are the low
//     and high nibbles of qs bytes 4g..4g+3, one Q4 word. x comes in that order (lmoe_to_gemm_f16), gate/up writes
//     h in it, and down reads it; results are the same sums, in another order;
//   * Q4_0 (k_grouped_q4_0): A and the raw weight units go global -> LDS directly (global_load_lds, no registers,
//     no VALU), two K steps ahead through a ring of three LDS stages, one barrier a step. Q4_K (k_grouped_q4_k):
//     thread t loads the unit of tile feature t into registers one step ahead and repacks it with its scales;
//   * the weights are the MFMA's first operand, so each lane ends with 4 consecutive output features of one row;
//     gate/up tiles hold 128 gate and 128 up features (a wavefront: 32 of each, the same ones), SwiGLU happens in
//     registers and h leaves as f16 in grouped row order. Down writes y [R][H] (f16 or f32) in grouped order.
// Operands are f16 with fp32 accumulation. A single rounding of (q - 8) d to f16 keeps the layer well inside the
// 2e-3 relative L2 bar; bf16 operands would not.
#include <cstdlib>
#include <type_traits>

#include "lmoe_common.h"

namespace lmoe {

template <int N>
using IC = std::integral_constant<int, N>;

// f(IC<0>), f(IC<1>), ..., f(IC<N - 1>): a loop whose index is a compile-time constant in the body
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
  if constexpr (I < N) {
    f(IC<I>{});
    static_for<I + 1, N>(f);
  }
}

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int GM = 128;  // rows a tile (the grouping kernel's bm)
constexpr int GN = 256;  // weight rows a tile (gate/up: 128 gate + 128 up features; down: 256 outputs)
constexpr int GK = 64;   // K a step (one 64-weight unit of every weight row)
constexpr int kThreads = 256;
constexpr int kTileMask = (1 << 20) - 1;

enum { MODE_GATE_UP = 0, MODE_DOWN = 1 };

// 16-byte chunk c (0..7) of A row r in a stage: rows are 128 bytes, chunks XOR-swizzled by the row's low 3 bits
__device__ __forceinline__ int achunk(int r, int c) { return r * 8 + (c ^ (r & 7)); }


// two f16 (1024 + q) from a byte-wise masked word: {q0, q1} or {q2, q3}
__device__ __forceinline__ uint32_t magic_pair(uint32_t nib, uint32_t sel) {
  return __builtin_amdgcn_perm(0x64646464u, nib, sel);
}
constexpr uint32_t kSel01 = 0x04010400u, kSel23 = 0x04030402u;

// An MFMA lane's 8 f16 weights from its nibble word x (low nibbles: K positions 0-3 of the lane group, high
// nibbles: 4-7). Q4_0: w = ((1024 + q) - 1032) d, d = the selected half of sw. Q4_K: sw = {f16(d sc), f16(dmin m)},
// w = fma((1024 + q) - 1024, d sc, -dmin m) (q exact, one rounding).
template <int TB>
__device__ __forceinline__ half8 decode8(uint32_t x, uint32_t sw, int half) {
  const uint32_t lo = x & 0x0F0F0F0Fu, hi = (x >> 4) & 0x0F0F0F0Fu;
  const h2_t p[4] = {__builtin_bit_cast(h2_t, magic_pair(lo, kSel01)), __builtin_bit_cast(h2_t, magic_pair(lo, kSel23)),
                     __builtin_bit_cast(h2_t, magic_pair(hi, kSel01)), __builtin_bit_cast(h2_t, magic_pair(hi, kSel23))};
  h2_t bias, scale, sub;
  if (TB == LMOE_Q4_0) {
    const _Float16 d = __builtin_bit_cast(h2_t, sw)[half];
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
  for (int i = 0; i < 4; ++i)
    o[i] = TB == LMOE_Q4_0 ? __builtin_bit_cast(uint32_t, (p[i] - bias) * scale)
                           : __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(p[i] - bias, scale, -sub));
  return __builtin_bit_cast(half8, u32x4{o[0], o[1], o[2], o[3]});
}

// Tile bookkeeping shared by both kernels
struct Tile {
  int e, nt, row0, rows, kpart;
};

// XCD-aware remap: workgroup `wid` runs on XCD wid % 8; XCD x gets logical work [start_x, start_x + count_x).
// Returns false for workgroups past the device-side work count.
// ksplit > 1: each (tile, n-tile) is worked by ksplit workgroups, one a slice of K (t->kpart), next to each other
// in the logical order.
template <int GMT = GM>
__device__ __forceinline__ bool tile_of(const uint32_t *offsets, const uint32_t *tiles, const uint32_t *n_tiles,
                                        int n_ntile, Tile *t, int ksplit = 1) {
  const uint32_t W = n_tiles[0] * uint32_t(n_ntile) * uint32_t(ksplit);
  const uint32_t wid = blockIdx.x;
  if (wid >= W) return false;
  const uint32_t q8 = W >> 3, r8 = W & 7, xcd = wid & 7;
  const uint32_t logical0 = xcd * q8 + min(xcd, r8) + (wid >> 3);
  t->kpart = int(logical0 % uint32_t(ksplit));
  const uint32_t logical = logical0 / uint32_t(ksplit);
  const uint32_t tile = tiles[logical / uint32_t(n_ntile)];
  t->nt = int(logical % uint32_t(n_ntile));
  t->e = int(tile >> 20);
  t->row0 = int(offsets[t->e]) + int(tile & kTileMask) * GMT;
  t->rows = min(GMT, int(offsets[t->e + 1]) - t->row0);
  return true;
}

// Tile features of a wavefront's 4 fragments: gate/up: gate 32 w + 16 nb (nb < 2), up 128 + 32 w + 16 (nb - 2)
// (the same intermediate features); down: 64 w + 16 nb
template <int MODE>
__device__ __forceinline__ int frag_feature(int wave, int nb) {
  return MODE == MODE_GATE_UP ? (nb < 2 ? 32 * wave + 16 * nb : GN / 2 + 32 * wave + 16 * (nb - 2))
                              : 64 * wave + 16 * nb;
}

// Two f16 of a, b packed in one word
__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
  return __builtin_bit_cast(uint32_t, h2_t{_Float16(a), _Float16(b)});
}

// acc[nb][mb][r] = D[tile feature frag_feature(nb) + 4 g + r][tile row 16 mb + fr]. Every store is 16 bytes:
//   * gate/up: h (f16, K order) = silu(gate) * up. A lane's features 4g..4g+3 of fragments 0 and 1 (32 w + 4g.. and
//     32 w + 16 + 4g.. of the n-tile) sit at K-order positions 8g..8g+3 and 8g+4..8g+7 of their 32-block: one store;
//   * down, f16: fragments nb and nb + 1 meet through one permlane16 swap a word: lane group g then holds 8
//     consecutive features, of fragment nb + (g & 1), from 8 (g >> 1) on, so a row's 32 features of the pair go out
//     as one 64-byte run; f32: each fragment's 4 features as they are.
// Called by every lane of the workgroup (the swaps read the lanes 16 away); rows past the tile's end store nothing.
template <int MODE, int MB = 8>
__device__ __forceinline__ void store_tile(f32x4 (&acc)[4][MB], const Tile &t, int wave, int fr, int g, void *out,
                                           int ldo, int odt) {
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int m = 16 * mb + fr;
    const bool ok = m < t.rows;
    const size_t o = size_t(t.row0 + (ok ? m : 0)) * ldo;
    if (MODE == MODE_GATE_UP) {
      uint32_t v[4];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int r = 0; r < 2; ++r)
          v[2 * nb + r] = pack_h2(silu_mul_h(acc[nb][mb][2 * r], acc[nb + 2][mb][2 * r]),
                                  silu_mul_h(acc[nb][mb][2 * r + 1], acc[nb + 2][mb][2 * r + 1]));
      const int n0 = t.nt * (GN / 2) + frag_feature<MODE>(wave, 0);  // a multiple of 32
      if (ok) *reinterpret_cast<u32x4 *>(static_cast<_Float16 *>(out) + o + n0 + 8 * g) = u32x4{v[0], v[1], v[2], v[3]};
    } else if (odt == LMOE_F32) {
      if (ok) {
#pragma unroll
        for (int nb = 0; nb < 4; ++nb)
          *reinterpret_cast<f32x4 *>(static_cast<float *>(out) + o + t.nt * GN + frag_feature<MODE>(wave, nb) +
                                     4 * g) = acc[nb][mb];
      }
    } else {
#pragma unroll
      for (int pr = 0; pr < 2; ++pr) {
        const int nb = 2 * pr;
        const auto s0 = __builtin_amdgcn_permlane16_swap(pack_h2(acc[nb][mb][0], acc[nb][mb][1]),
                                                         pack_h2(acc[nb + 1][mb][0], acc[nb + 1][mb][1]), false, false);
        const auto s1 = __builtin_amdgcn_permlane16_swap(pack_h2(acc[nb][mb][2], acc[nb][mb][3]),
                                                         pack_h2(acc[nb + 1][mb][2], acc[nb + 1][mb][3]), false, false);
        const uint32_t a0 = s0[0], b0 = s0[1], a1 = s1[0], b1 = s1[1];
        const int n = t.nt * GN + frag_feature<MODE>(wave, nb + (g & 1)) + 8 * (g >> 1);
        if (ok) *reinterpret_cast<u32x4 *>(static_cast<_Float16 *>(out) + o + n) = u32x4{a0, a1, b0, b1};
      }
    }
  }
}

// ---- the stream layout -----------------------------------------------------------------------------------------
//
// A second copy of a Q4 expert matrix [E][rows][row bytes] (rows % 128 == 0), for the grouped GEMMs of resident
// layers: the same bytes, ordered so that what a GEMM step copies for a block of 128 features is contiguous (in the
// GGUF order each feature's 32 or 36 bytes of a step sit a row apart, and copies of such pieces run at ~4.9 TB/s
// against ~6.2 for contiguous ones). Blocks in the order [expert][feature block fb of 128][K block]:
//   Q4_0, a K block = one 64-weight step (two GGUF blocks, 36 bytes a feature), 4,608 bytes: granule q (16 bytes,
//     q < 256) = half (q / 16) % 2 (bytes 16 h .. 16 h + 15 of the 36) of block feature 16 (q / 32) + q % 16, then
//     the 128 features' bytes 32..35, 4 a feature;
//   Q4_K, a K block = one super-block (256 weights, 4 steps), 18,432 bytes: the 128 features' 16-byte headers, then
//     for each of the 4 steps pr, granule q = half (q / 16) % 2 of block feature 16 (q / 32) + q % 16's step bytes
//     (super-block bytes 16 + 32 pr + 16 h .. + 15).
// The granule order is the LDS order of a GEMM stage, so a wavefront's copies of a step read one kilobyte each.
constexpr int kSlQ0 = 4608, kSlQK = 18432;

// One thread a dword of the stream copy: where it comes from in the GGUF matrix.
template <int TQ>
__global__ void __launch_bounds__(256) k_stream_repack(const uint32_t *src, int rows, int row_dw, int nkb,
                                                       long long n_dw, uint32_t *dst) {
  const long long d = (long long)blockIdx.x * 256 + threadIdx.x;
  if (d >= n_dw) return;
  constexpr int BDW = (TQ == LMOE_Q4_K ? kSlQK : kSlQ0) / 4;
  const long long blk = d / BDW;
  const int o = int(d - blk * BDW);
  const int kb = int(blk % nkb);
  const long long efb = blk / nkb;  // expert * (rows / 128) + fb
  const int fb = int(efb % (rows / 128));
  const long long e = efb / (rows / 128);
  int feature, byte;
  if (TQ == LMOE_Q4_0) {
    if (o < 1024) {
      const int q = o >> 2, w = o & 3;
      feature = 16 * (q >> 5) + (q & 15);
      byte = 36 * kb + 16 * ((q >> 4) & 1) + 4 * w;
    } else {
      feature = o - 1024;
      byte = 36 * kb + 32;
    }
  } else {
    if (o < 512) {
      feature = o >> 2;
      byte = 144 * kb + 4 * (o & 3);
    } else {
      const int o2 = o - 512, pr = o2 >> 10, r = o2 & 1023, q = r >> 2, w = r & 3;
      feature = 16 * (q >> 5) + (q & 15);
      byte = 144 * kb + 16 + 32 * pr + 16 * ((q >> 4) & 1) + 4 * w;
    }
  }
  dst[d] = src[(e * rows + fb * 128 + feature) * row_dw + byte / 4];
}

// ---- Q4_0: global -> LDS directly, three stages ------------------------------------------------------------------

// Per tile-row count GMT (128, or 32 for groups of few rows): A tile bytes a stage, the stage, A copies a lane.
template <int GMT> constexpr int q0_astage() { return GMT * 128; }
constexpr int kQ0WHead = GN * 32;               // the first 32 bytes of every unit (words 0-7), 32 a feature
template <int GMT> constexpr int q0_stage() { return q0_astage<GMT>() + GN * 36; }  // + word 8 of every unit
template <int GMT> constexpr int q0_dma_a() { return GMT * 128 / 1024 / 4; }      // 16-byte A copies a lane a step
constexpr int kQ0DmaW = GN * 32 / 1024 / 4;     // 16-byte unit-head copies a lane a step (2), plus one 4-byte copy

// A wavefront-uniform pointer held in scalar registers (the copy instructions take their base there)
template <typename P>
__device__ __forceinline__ P *uniform(P *p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(v)), hi = __builtin_amdgcn_readfirstlane(uint32_t(v >> 32));
  return reinterpret_cast<P *>((uint64_t(hi) << 32) | lo);
}

// One wavefront-wide global -> LDS copy: lane l's `BYTES` (4 or 16) at base + voff land at LDS address
// lds + l * BYTES (global_load_lds_dwordx3 would also step 16 bytes a lane). M0 carries the LDS address; nothing
// else in these kernels uses M0.
template <int BYTES>
__device__ __forceinline__ void dma(const void *base_any, uint32_t voff, uint32_t lds) {
  const void *base = uniform(base_any);
  if (BYTES == 16)
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "s"(lds) : "memory");
  else
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(base), "s"(lds) : "memory");
}

// The A copies of a tile whose rows end early: copy i of wavefront w (D copies a wavefront a step) moves tile rows
// [8 (D w + i), +8); bit i of the mask says whether any of them is a row of the tile. A copy of rows past the end
// becomes a 4-byte copy of one address into the same place (the rows' LDS bytes are never stored: their output
// rows are masked), so every wavefront still issues the same number of copies a step and the counted waits hold,
// while the padding rows of a short group (~40 rows in a 64-row tile, ~5 in a 32-row one) cost no A bytes.
template <int D>
__device__ __forceinline__ uint32_t a_live_mask(int wave, int rows) {
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < D; ++i) m |= (8 * (D * wave + i) < rows ? 1u : 0u) << i;
  return __builtin_amdgcn_readfirstlane(m);
}

__device__ __forceinline__ void dma_a(const _Float16 *ab, uint32_t off, uint32_t lds, uint32_t live) {
  if (live)
    dma<16>(ab, off, lds);
  else
    dma<4>(ab, 0u, lds);
}

// s_barrier with compiler memory fences on both sides: the intrinsic alone does not order memory accesses, and
// __syncthreads' release fence would wait for every copy in flight, including the ones meant to stay in flight
__device__ __forceinline__ void barrier_lds() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// s_waitcnt on the vector-memory counter only (the copies this wavefront issued), N outstanding at most
template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Where lane (fr, g) of a wavefront finds its 4 weight fragments in a Q4_0 stage (the same for every tile). Lane
// (fr, g) of fragment nb decodes tile feature f = frag_feature(nb) + fr's unit: block 0 qs bytes 4g..+3 (unit bytes
// 2 + 4g.., straddling words g and g + 1), block 1 qs bytes 4g..+3 (word 5 + g; word 8 sits in the tail area),
// d0 / d1 in the low half of word 0 / the high half of word 4. Byte offsets in a stage: the feature's first half at
// head[nb], its second half 256 bytes on; word g + 1 at head[nb] + w1_of; block 1's word at blk1[nb].
struct Q0Lane {
  int head[4], blk1[4], w1_of;
};

template <int MODE, int GMT>
__device__ __forceinline__ Q0Lane q0_lane(int wave, int fr, int g) {
  Q0Lane L;
  L.w1_of = g < 3 ? 4 * g + 4 : 256;
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) {
    const int f = frag_feature<MODE>(wave, nb) + fr;
    L.head[nb] = q0_astage<GMT>() + 512 * (f >> 4) + 16 * (f & 15);
    L.blk1[nb] = g < 3 ? L.head[nb] + 256 + 4 * (1 + g) : q0_astage<GMT>() + kQ0WHead + 4 * f;
  }
  return L;
}

// One K step of a wavefront out of the Q4_0 stage at st into acc. The MFMA order is written out by hand. The
// step's 8 weight fragments (K slice ks = i / 4, fragment nb = i % 4) go in turn; fragment i's 8 MFMAs issue in
// pairs with a quarter of fragment i + 1's decode (4 VALU) between pairs, so the decode issues while the matrix
// core works; fragment i + 2's weight word is read from LDS one fragment ahead of its decode and the second K
// slice's A fragments two fragments ahead of their use. sched_barrier keeps the compiler from regrouping them.
// QN: the 32-row pairs of fragments the tile has rows in (a tile's last m-tile is often short): the MFMAs and A
// reads of empty pairs are left out.
// The step body, over any weight layout: word(i) / scale(i) give fragment i's nibble word and the word holding its
// block scale (low half for K slice 0, high half for K slice 1); sa is the step's A stage.
template <int QN, int MB, typename Word, typename Scale>
__device__ __forceinline__ void q0_mfma_step(const uint8_t *sa, Word word, Scale scale, int fr, int g,
                                             f32x4 (&acc)[4][MB]) {
  __builtin_amdgcn_s_setprio(1);  // the other workgroup's wavefront on this SIMD yields while this one multiplies
  const u32x4 *as = reinterpret_cast<const u32x4 *>(sa);
  const h2_t bias = {_Float16(1032.0f), _Float16(1032.0f)};
  half8 xf[2][8];
#pragma unroll
  for (int mb = 0; mb < 2 * QN; ++mb) xf[0][mb] = __builtin_bit_cast(half8, as[achunk(16 * mb + fr, g)]);
  uint32_t xw[8], sw[8];  // fully unrolled: each element lives in its own registers
  xw[0] = word(0);
  sw[0] = scale(0);
  xw[1] = word(1);
  sw[1] = scale(1);
  u32x4 wcur = __builtin_bit_cast(u32x4, decode8<LMOE_Q4_0>(xw[0], sw[0], 0));
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int ks = i / 4, nb = i % 4;
    if (i + 2 < 8) {
      xw[i + 2] = word(i + 2);
      sw[i + 2] = scale(i + 2);
    }
    if (i == 2) {
#pragma unroll
      for (int mb = 0; mb < 2 * QN; ++mb) xf[1][mb] = __builtin_bit_cast(half8, as[achunk(16 * mb + fr, 4 + g)]);
    }
    const int n = i + 1 < 8 ? i + 1 : 7;  // the next fragment (a repeat of the last, unused, after it)
    const _Float16 d = __builtin_bit_cast(h2_t, sw[n])[n / 4];
    const h2_t dd = {d, d};
    uint32_t lo = 0, hi = 0;
    u32x4 wnext;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (q < QN) {
        acc[nb][2 * q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, wcur), xf[ks][2 * q],
                                                                 acc[nb][2 * q], 0, 0, 0);
        acc[nb][2 * q + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, wcur),
                                                                     xf[ks][2 * q + 1], acc[nb][2 * q + 1], 0, 0, 0);
      }
      if (i + 1 < 8) {
        if (q == 0) {
          lo = xw[n] & 0x0F0F0F0Fu;
          hi = (xw[n] >> 4) & 0x0F0F0F0Fu;
        }
        const uint32_t p = magic_pair(q < 2 ? lo : hi, q % 2 == 0 ? kSel01 : kSel23);
        wnext[q] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2_t, p) - bias) * dd);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (i + 1 < 8) wcur = wnext;
  }
  __builtin_amdgcn_s_setprio(0);
}

template <int QN, int MB>
__device__ __forceinline__ void q0_step(const uint8_t *st, const Q0Lane &L, int fr, int g, f32x4 (&acc)[4][MB]) {
  auto at = [&](int byte) -> uint32_t { return *reinterpret_cast<const uint32_t *>(st + byte); };
  auto word = [&](int i) -> uint32_t {
    const int ks = i / 4, nb = i % 4;
    return ks == 0 ? __builtin_amdgcn_alignbyte(at(L.head[nb] + L.w1_of), at(L.head[nb] + 4 * g), 2) : at(L.blk1[nb]);
  };
  auto scale = [&](int i) -> uint32_t { return at(L.head[i % 4] + 256 * (i / 4)); };
  q0_mfma_step<QN, MB>(st, word, scale, fr, g, acc);
}

// ---- Q4_0 on the GGUF layout, two units a step -------------------------------------------------------------------
//
// In the GGUF layout a one-unit step copies 36 bytes of each of 256 weight rows, a 128-byte line a row for 32 of its
// bytes, and the line is gone from L1 before the next step wants the rest of it (rocprofv3 on cfg4's 32-row tiles:
// 5.3x the L1-to-L2 requests of the stream copies, the texture unit stalled on L1 tags). A step of two units (K 128)
// copies 72 contiguous bytes a row: a 16-byte copy instruction takes 16 rows x 64 bytes (four lanes a row), a 4-byte
// one 32 rows x 8 bytes. LDS a stage: the one-unit kernel's A stage twice (K 0-63, 64-127), then wavefront w's copy
// rows (tile features 64 w .. 64 w + 63) as 4 blocks of 16 rows x 64 bytes, each padded to kW2Blk bytes, then 8
// blocks of 32 rows x 8 bytes (piece bytes 64-71). Feature 16 q + 4 i + j (q, i, j < 4) of a wavefront sits in block
// i, slot 4 q + j, so the 16 features of an MFMA fragment (q fixed) lie kW2Blk i + 64 j apart: 16 different groups
// of four banks. Same arithmetic as two one-unit steps, so the same bits.
constexpr int kW2Blk = 1040, kW2X4 = 4 * 4 * kW2Blk, kW2Dw = 8 * 256;
template <int GMT> constexpr int q0w2_stage() { return 2 * q0_astage<GMT>() + kW2X4 + kW2Dw; }

// Lane (fr, g)'s addresses in a two-unit stage for fragment nb: x = the feature's 64-byte run, xg = x + 4 g,
// b1 = unit 1's block-1 word 5 + g (piece word 14 + g: in the run for g < 2, else in the 8-byte tail)
struct Q0Lane2 {
  int x[4], xg[4], b1[4];
};

// base: the byte offset of the weight area (the 16-byte blocks, then the 8-byte tails) from the stage's start
template <int MODE>
__device__ __forceinline__ Q0Lane2 q0_lane2(int wave, int fr, int g, int base) {
  Q0Lane2 L;
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) {
    const int f = frag_feature<MODE>(wave, nb) + fr;
    const int cw = f >> 6, fl = f & 63, q = fl >> 4, i = (fl >> 2) & 3, j = fl & 3;
    const int x = base + cw * 4 * kW2Blk + i * kW2Blk + 64 * (4 * q + j);
    const int d = base + kW2X4 + (2 * cw + (fl >> 5)) * 256 + 8 * (fl & 31);
    L.x[nb] = x;
    L.xg[nb] = x + 4 * g;
    L.b1[nb] = g < 2 ? x + 4 * (14 + g) : d + 4 * (g - 2);
  }
  return L;
}

// Unit U (0, 1) of a two-unit weight stage at sw (unit words w are piece words 9 U + w) against the A stage at sa
template <int QN, int MB, int U>
__device__ __forceinline__ void q0_step_pair(const uint8_t *sa, const uint8_t *sw, const Q0Lane2 &L, int fr, int g,
                                             f32x4 (&acc)[4][MB]) {
  auto at = [&](int byte) -> uint32_t { return *reinterpret_cast<const uint32_t *>(sw + byte); };
  auto word = [&](int i) -> uint32_t {
    const int ks = i / 4, nb = i % 4;
    if (ks == 0) return __builtin_amdgcn_alignbyte(at(L.xg[nb] + 36 * U + 4), at(L.xg[nb] + 36 * U), 2);
    return U == 0 ? at(L.xg[nb] + 20) : at(L.b1[nb]);
  };
  auto scale = [&](int i) -> uint32_t { return at(L.x[i % 4] + 36 * U + 16 * (i / 4)); };
  q0_mfma_step<QN, MB>(sa, word, scale, fr, g, acc);
}

// Unit U of a two-unit stage (A of both units, then the weights, at st)
template <int QN, int MB, int U>
__device__ __forceinline__ void q0_step2(const uint8_t *st, const Q0Lane2 &L, int fr, int g, f32x4 (&acc)[4][MB]) {
  q0_step_pair<QN, MB, U>(st + U * q0_astage<MB * 16>(), st, L, fr, g, acc);
}

// Grid: n_ntile * max_tiles workgroups of 256 threads, two a CU. GATE_UP: n-tile j covers intermediate features
// 128 j .. 128 j + 127 (tile features 0..127 their gate rows, 128..255 their up rows), K = H, A rows
// x[order[p] / topk], out h [R][I] f16. DOWN: n-tile j covers output features 256 j .., K = I, A rows h[p], out
// y [R][H] in odt (F16 / F32). Host guarantees: K % 64 == 0, rows x K x 2 and the expert's weight block under 4 GiB.
// GMT: tile rows (the grouping's bm): 128 with NST = 3 stages, 64 with 4, or 32 with 3 or 5 for groups of few rows,
// where the kernel streams weights (5: more steps in flight; 3: four workgroups a CU instead of two).
// ksplit > 1 (32-row tiles): workgroup kpart takes K steps [kpart nk / ksplit, +nk / ksplit) and writes its fp32
// sums to ws[kpart][row][feature] (features: gate/up = gate 0..I-1, up I..2I-1; down = 0..H-1; ldw of them a row,
// R rows a slice); k_splitk_finish adds the slices and applies the epilogue.
template <int MODE, int GMT = GM, int NST = 3, bool SL = false>
__global__ void __launch_bounds__(kThreads, 2)
k_grouped_q4_0(const _Float16 *a_src, int topk, const uint32_t *order, const uint32_t *offsets,
               const uint32_t *tiles, const uint32_t *n_tiles, int n_ntile, const uint8_t *w0, const uint8_t *w1,
               int K, int n_rows, void *out, int ldo, int odt, int ksplit = 1, float *ws = nullptr, int R = 0,
               int ldw = 0) {
  constexpr int kQ0AStage = q0_astage<GMT>(), kQ0Stage = q0_stage<GMT>(), kQ0DmaA = q0_dma_a<GMT>();
  constexpr int MB = GMT / 16, QMAX = GMT / 32;
  static_assert(kQ0DmaA >= 1 && NST >= 3, "tile and pipeline shape");
  __shared__ __attribute__((aligned(16))) uint8_t lds[NST * kQ0Stage];
  Tile t;
  if (!tile_of<GMT>(offsets, tiles, n_tiles, n_ntile, &t, ksplit)) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 15, g = lane >> 4;
  const uint32_t wrow = 36u * uint32_t(K / 64);
  const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>(lds));

  // A: wavefront w's load i fills LDS bytes [1024 (4 w + i), +1024) of a stage: 16-byte granule q = 64 (4 w + i) +
  // lane holds chunk (q % 8) ^ (r & 7) of tile row r = q / 8. Rows past the tile's end read its first row.
  uint32_t a_off[kQ0DmaA];
#pragma unroll
  for (int i = 0; i < kQ0DmaA; ++i) {
    const int q = 64 * (kQ0DmaA * wave + i) + lane, r = q >> 3, c = (q & 7) ^ (r & 7);
    const int p = t.row0 + (r < t.rows ? r : 0);
    const uint32_t row = MODE == MODE_GATE_UP ? order[p] / uint32_t(topk) : uint32_t(p);
    a_off[i] = row * uint32_t(K) * 2u + 16u * uint32_t(c);
  }
  const uint32_t a_live = a_live_mask<kQ0DmaA>(wave, t.rows);
  // weights: wavefront w covers tile features 64 w .. 64 w + 63 (gate/up: waves 0-1 gate rows, 2-3 up rows).
  // Its 16-byte copy i fills bytes [1024 (2 w + i), +1024) of the stage's head area: granule q = 64 (2 w + i) +
  // lane is half h = (q / 16) % 2 (words 4h .. 4h + 3) of tile feature f = 16 (q / 32) + q % 16. So each group of
  // 16 features keeps its 16 first halves in one 256-byte row and its 16 second halves in the next: the 16
  // features an MFMA fragment reads sit in 16 different 16-byte columns, and its 64 lanes in 64 different banks.
  // Its 4-byte copy puts word 8 of tile feature 64 w + lane at 4 f of the tail area.
  const uint8_t *wbase;
  uint32_t w_off[kQ0DmaW + 1];
  if constexpr (SL) {
    // the stream layout (k_stream_repack): wavefront w's 128-feature block fb, one 4,608-byte block a K step: the
    // granules and tail words this wavefront copies are one contiguous run of each
    const uint8_t *m = MODE == MODE_GATE_UP && wave >= 2 ? w1 : w0;
    const int fb = MODE == MODE_GATE_UP ? t.nt : 2 * t.nt + (wave >> 1);
    wbase = m + (size_t(t.e) * (n_rows / 128) + fb) * size_t(K / GK) * kSlQ0;
#pragma unroll
    for (int i = 0; i < kQ0DmaW; ++i) w_off[i] = 16u * uint32_t(64 * (kQ0DmaW * (wave & 1) + i) + lane);
    w_off[kQ0DmaW] = 4096u + 4u * uint32_t(64 * (wave & 1) + lane);
  } else {
    const uint8_t *m = MODE == MODE_GATE_UP && wave >= 2 ? w1 : w0;
    const int row_base = MODE == MODE_GATE_UP ? t.nt * (GN / 2) - (wave >= 2 ? GN / 2 : 0) : t.nt * GN;
    wbase = m + (size_t(t.e) * n_rows) * wrow;
#pragma unroll
    for (int i = 0; i < kQ0DmaW; ++i) {
      const int q = 64 * (kQ0DmaW * wave + i) + lane;
      w_off[i] = uint32_t(row_base + 16 * (q >> 5) + (q & 15)) * wrow + 16u * uint32_t((q >> 4) & 1);
    }
    w_off[kQ0DmaW] = uint32_t(row_base + 64 * wave + lane) * wrow + 32u;
  }
  const int nk = K / GK / ksplit, k0 = t.kpart * nk;  // this workgroup's K steps: k0 .. k0 + nk - 1
  auto issue = [&](int kk) {  // step kk (of the slice) into stage kk % NST
    const uint32_t st = lds0 + uint32_t(kk % NST) * kQ0Stage;
    const _Float16 *ab = a_src + size_t(k0 + kk) * GK;
#pragma unroll
    for (int i = 0; i < kQ0DmaA; ++i)
      dma_a(ab, a_off[i], __builtin_amdgcn_readfirstlane(st + 1024u * uint32_t(kQ0DmaA * wave + i)), a_live >> i & 1u);
    const uint8_t *wb = wbase + size_t(k0 + kk) * (SL ? kSlQ0 : 36);
#pragma unroll
    for (int i = 0; i < kQ0DmaW; ++i)
      dma<16>(wb, w_off[i], __builtin_amdgcn_readfirstlane(st + kQ0AStage + 1024u * uint32_t(kQ0DmaW * wave + i)));
    dma<4>(wb, w_off[kQ0DmaW], __builtin_amdgcn_readfirstlane(st + kQ0AStage + kQ0WHead + 256u * uint32_t(wave)));
  };

  f32x4 acc[4][MB];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const Q0Lane ql = q0_lane<MODE, GMT>(wave, fr, g);
  // the stage as a compile-time index: every LDS address of a step is then a lane offset plus an immediate
  auto compute = [&](auto s, auto qn) {
    q0_step<decltype(qn)::value, MB>(lds + decltype(s)::value * kQ0Stage, ql, fr, g, acc);
  };

  // Step kk: the copies of step kk + NST - 1 go out, step kk multiplies out of its stage, then each wavefront waits
  // for its own copies of step kk + 1 (the counter counts in issue order: the copies of the steps after kk + 1 may
  // still be out) and the barrier publishes the stage. The barrier also tells the next step that stage kk % NST,
  // which it refills, has been read by every wavefront.
  constexpr int C = kQ0DmaA + kQ0DmaW + 1;  // copies a lane a step
  static_assert(NST <= 5 && 3 * C <= 63, "the wait counts below");
  auto wait_steps = [&](int later) {  // until at most `later` steps' copies are still out
    if (later <= 0)
      wait_vm<0>();
    else if (later == 1)
      wait_vm<C>();
    else if (later == 2)
      wait_vm<2 * C>();
    else
      wait_vm<3 * C>();
  };
  const int pre = min(NST - 1, nk);
  for (int j = 0; j < pre; ++j) issue(j);
  wait_steps(pre - 1);
  barrier_lds();
  auto run = [&](auto qn) {
    for (int kb = 0; kb < nk; kb += NST) {  // NST steps a pass, so step kb + j reads stage j
      static_for<0, NST>([&](auto j) {
        const int kk = kb + decltype(j)::value;
        if (kk < nk) {
          if (kk + NST - 1 < nk) issue(kk + NST - 1);
          compute(j, qn);
          if (kk + 1 < nk) {
            wait_steps(min(kk + NST - 1, nk - 1) - (kk + 1));
            barrier_lds();
          }
        }
      });
    }
  };
  if constexpr (QMAX == 1) {
    run(IC<1>{});
  } else if constexpr (QMAX == 2) {
    if (t.rows <= 32)  // uniform across the workgroup
      run(IC<1>{});
    else
      run(IC<2>{});
  } else {
    switch ((t.rows + 31) / 32) {  // uniform across the workgroup
      case 1: run(IC<1>{}); break;
      case 2: run(IC<2>{}); break;
      case 3: run(IC<3>{}); break;
      default: run(IC<4>{}); break;
    }
  }
  if (ksplit > 1) {
    // fp32 partial sums of this K slice: 4 consecutive features of one row a store
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int m = 16 * mb + fr;
      if (m >= t.rows) continue;
      float *wrow = ws + (size_t(t.kpart) * R + t.row0 + m) * ldw;
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        const int f = frag_feature<MODE>(wave, nb) + 4 * g;
        const int n = MODE == MODE_GATE_UP ? (f < GN / 2 ? t.nt * (GN / 2) + f : ldw / 2 + t.nt * (GN / 2) + f - GN / 2)
                                           : t.nt * GN + f;
        *reinterpret_cast<f32x4 *>(wrow + n) = acc[nb][mb];
      }
    }
    return;
  }
  store_tile<MODE, MB>(acc, t, wave, fr, g, out, ldo, odt);
}

// k_grouped_q4_0 on the GGUF layout with two-unit steps (K 128, the stage above): grid, arguments and results as
// k_grouped_q4_0<MODE, GMT> (the same bits); host guarantees K % (128 ksplit) == 0. NST = 3 stages (79 KB, two
// workgroups a CU) or 2 (53 KB, three a CU: the next step's copies fly while this one multiplies).
template <int MODE, int GMT, int NST>
__global__ void __launch_bounds__(kThreads, NST == 2 ? 3 : 2)
k_grouped_q4_0_w2(const _Float16 *a_src, int topk, const uint32_t *order, const uint32_t *offsets,
                  const uint32_t *tiles, const uint32_t *n_tiles, int n_ntile, const uint8_t *w0, const uint8_t *w1,
                  int K, int n_rows, void *out, int ldo, int odt, int ksplit = 1, float *ws = nullptr, int R = 0,
                  int ldw = 0) {
  constexpr int kAStage = q0_astage<GMT>(), kStage = q0w2_stage<GMT>(), kDmaA = q0_dma_a<GMT>();
  constexpr int MB = GMT / 16, QMAX = GMT / 32;
  static_assert(kDmaA >= 1 && (NST == 2 || NST == 3) && NST * kStage <= 81920, "tile and pipeline shape");
  __shared__ __attribute__((aligned(16))) uint8_t lds[NST * kStage];
  Tile t;
  if (!tile_of<GMT>(offsets, tiles, n_tiles, n_ntile, &t, ksplit)) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 15, g = lane >> 4;
  const uint32_t wrow = 36u * uint32_t(K / 64);
  const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>(lds));

  // A: as in k_grouped_q4_0, once for each 64-K half of the step
  uint32_t a_off[kDmaA];
#pragma unroll
  for (int i = 0; i < kDmaA; ++i) {
    const int q = 64 * (kDmaA * wave + i) + lane, r = q >> 3, c = (q & 7) ^ (r & 7);
    const int p = t.row0 + (r < t.rows ? r : 0);
    const uint32_t row = MODE == MODE_GATE_UP ? order[p] / uint32_t(topk) : uint32_t(p);
    a_off[i] = row * uint32_t(K) * 2u + 16u * uint32_t(c);
  }
  const uint32_t a_live = a_live_mask<kDmaA>(wave, t.rows);
  // weights: wavefront w copies tile features 64 w .. 64 w + 63 (gate/up: waves 0-1 gate rows, 2-3 up rows).
  // 16-byte copy i: lane l takes bytes 16 (l % 4) .. of the step's piece of feature 16 (s / 4) + 4 i + s % 4,
  // s = l / 4; 4-byte copy j: lane l takes piece bytes 64 + 4 (l % 2) of feature 32 j + l / 2.
  const uint8_t *m = MODE == MODE_GATE_UP && wave >= 2 ? w1 : w0;
  const int row_base = (MODE == MODE_GATE_UP ? t.nt * (GN / 2) - (wave >= 2 ? GN / 2 : 0) : t.nt * GN) + 64 * wave;
  const uint8_t *wbase = m + (size_t(t.e) * n_rows) * wrow;
  uint32_t w_off[4], d_off[2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int s = lane >> 2, fl = 16 * (s >> 2) + 4 * i + (s & 3);
    w_off[i] = uint32_t(row_base + fl) * wrow + 16u * uint32_t(lane & 3);
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) d_off[j] = uint32_t(row_base + 32 * j + (lane >> 1)) * wrow + 64u + 4u * uint32_t(lane & 1);
  const int nk = K / (2 * GK) / ksplit, k0 = t.kpart * nk;  // this workgroup's two-unit steps: k0 .. k0 + nk - 1
  auto issue = [&](int kk) {  // step kk (of the slice) into stage kk % NST
    const uint32_t st = lds0 + uint32_t(kk % NST) * kStage;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const _Float16 *ab = a_src + size_t(2 * (k0 + kk) + h) * GK;
#pragma unroll
      for (int i = 0; i < kDmaA; ++i)
        dma_a(ab, a_off[i], __builtin_amdgcn_readfirstlane(st + uint32_t(h * kAStage) + 1024u * uint32_t(kDmaA * wave + i)),
              a_live >> i & 1u);
    }
    const uint8_t *wb = wbase + size_t(k0 + kk) * 72;
    const uint32_t sw = st + 2u * kAStage;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      dma<16>(wb, w_off[i], __builtin_amdgcn_readfirstlane(sw + uint32_t(wave * 4 * kW2Blk + i * kW2Blk)));
#pragma unroll
    for (int j = 0; j < 2; ++j)
      dma<4>(wb, d_off[j], __builtin_amdgcn_readfirstlane(sw + uint32_t(kW2X4) + 256u * uint32_t(2 * wave + j)));
  };

  f32x4 acc[4][MB];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const Q0Lane2 ql = q0_lane2<MODE>(wave, fr, g, 2 * kAStage);
  auto compute = [&](auto s, auto qn) {
    const uint8_t *st = lds + decltype(s)::value * kStage;
    q0_step2<decltype(qn)::value, MB, 0>(st, ql, fr, g, acc);
    q0_step2<decltype(qn)::value, MB, 1>(st, ql, fr, g, acc);
  };

  constexpr int C = 2 * kDmaA + 6;  // copies a lane a step
  static_assert(3 * C <= 63, "the wait counts below");
  auto wait_steps = [&](int later) {  // until at most `later` steps' copies are still out
    if (later <= 0)
      wait_vm<0>();
    else if (later == 1)
      wait_vm<C>();
    else
      wait_vm<2 * C>();
  };
  const int pre = min(NST - 1, nk);
  for (int j = 0; j < pre; ++j) issue(j);
  wait_steps(pre - 1);
  barrier_lds();
  auto run = [&](auto qn) {
    for (int kb = 0; kb < nk; kb += NST) {
      static_for<0, NST>([&](auto j) {
        const int kk = kb + decltype(j)::value;
        if (kk < nk) {
          if (kk + NST - 1 < nk) issue(kk + NST - 1);
          compute(j, qn);
          if (kk + 1 < nk) {
            wait_steps(min(kk + NST - 1, nk - 1) - (kk + 1));
            barrier_lds();
          }
        }
      });
    }
  };
  if constexpr (QMAX == 1) {
    run(IC<1>{});
  } else if constexpr (QMAX == 2) {
    if (t.rows <= 32)
      run(IC<1>{});
    else
      run(IC<2>{});
  } else {
    switch ((t.rows + 31) / 32) {
      case 1: run(IC<1>{}); break;
      case 2: run(IC<2>{}); break;
      case 3: run(IC<3>{}); break;
      default: run(IC<4>{}); break;
    }
  }
  if (ksplit > 1) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int mrow = 16 * mb + fr;
      if (mrow >= t.rows) continue;
      float *wrw = ws + (size_t(t.kpart) * R + t.row0 + mrow) * ldw;
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        const int f = frag_feature<MODE>(wave, nb) + 4 * g;
        const int n = MODE == MODE_GATE_UP ? (f < GN / 2 ? t.nt * (GN / 2) + f : ldw / 2 + t.nt * (GN / 2) + f - GN / 2)
                                           : t.nt * GN + f;
        *reinterpret_cast<f32x4 *>(wrw + n) = acc[nb][mb];
      }
    }
    return;
  }
  store_tile<MODE, MB>(acc, t, wave, fr, g, out, ldo, odt);
}

// k_grouped_q4_0<MODE, GMT> on the GGUF layout for the tall tiles (128 or 64 rows, no split-K), with the weights
// staged two units at a time and A one unit at a time. A two-unit stage of A and weights for 128 rows (51 KB) leaves
// room for one stage at two workgroups a CU, so the ring is split: two A stages (one K step ahead) and two
// two-unit weight stages (the layout of k_grouped_q4_0_w2's weight area; one pair ahead). At step kk the A of step
// kk + 1 goes out, and on even kk the weights of pair kk / 2 + 1. The same arithmetic as k_grouped_q4_0: the same
// bits. Arguments as k_grouped_q4_0 (the split-K ones unused: one K slice). Host guarantees: K % 128 == 0, and
// those of k_grouped_q4_0.
constexpr int kP2WStage = kW2X4 + kW2Dw;  // a two-unit weight stage
template <int MODE, int GMT>
__global__ void __launch_bounds__(kThreads, 2)
k_grouped_q4_0_p2(const _Float16 *a_src, int topk, const uint32_t *order, const uint32_t *offsets,
                  const uint32_t *tiles, const uint32_t *n_tiles, int n_ntile, const uint8_t *w0, const uint8_t *w1,
                  int K, int n_rows, void *out, int ldo, int odt, int /*ksplit: 1*/, float * /*ws*/, int /*R*/,
                  int /*ldw*/) {
  constexpr int kAStage = q0_astage<GMT>(), kDmaA = q0_dma_a<GMT>();
  constexpr int kW = 2 * kAStage;  // the weight stages follow the two A stages
  constexpr int MB = GMT / 16, QMAX = GMT / 32;
  static_assert(kDmaA >= 1 && kW + 2 * kP2WStage <= 81920, "two workgroups a CU");
  __shared__ __attribute__((aligned(16))) uint8_t lds[kW + 2 * kP2WStage];
  Tile t;
  if (!tile_of<GMT>(offsets, tiles, n_tiles, n_ntile, &t)) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 15, g = lane >> 4;
  const uint32_t wrow = 36u * uint32_t(K / 64);
  const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>(lds));

  uint32_t a_off[kDmaA];  // A: as in k_grouped_q4_0
#pragma unroll
  for (int i = 0; i < kDmaA; ++i) {
    const int q = 64 * (kDmaA * wave + i) + lane, r = q >> 3, c = (q & 7) ^ (r & 7);
    const int p = t.row0 + (r < t.rows ? r : 0);
    const uint32_t row = MODE == MODE_GATE_UP ? order[p] / uint32_t(topk) : uint32_t(p);
    a_off[i] = row * uint32_t(K) * 2u + 16u * uint32_t(c);
  }
  const uint32_t a_live = a_live_mask<kDmaA>(wave, t.rows);
  // weights: as in k_grouped_q4_0_w2 (wavefront w copies tile features 64 w .. 64 w + 63)
  const uint8_t *m = MODE == MODE_GATE_UP && wave >= 2 ? w1 : w0;
  const int row_base = (MODE == MODE_GATE_UP ? t.nt * (GN / 2) - (wave >= 2 ? GN / 2 : 0) : t.nt * GN) + 64 * wave;
  const uint8_t *wbase = m + (size_t(t.e) * n_rows) * wrow;
  uint32_t w_off[4], d_off[2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int s = lane >> 2, fl = 16 * (s >> 2) + 4 * i + (s & 3);
    w_off[i] = uint32_t(row_base + fl) * wrow + 16u * uint32_t(lane & 3);
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) d_off[j] = uint32_t(row_base + 32 * j + (lane >> 1)) * wrow + 64u + 4u * uint32_t(lane & 1);
  const int nk = K / GK, np = nk / 2;
  auto issue_a = [&](int kk) {  // step kk's A into A stage kk % 2
    const uint32_t st = lds0 + uint32_t(kk & 1) * kAStage;
    const _Float16 *ab = a_src + size_t(kk) * GK;
#pragma unroll
    for (int i = 0; i < kDmaA; ++i)
      dma_a(ab, a_off[i], __builtin_amdgcn_readfirstlane(st + 1024u * uint32_t(kDmaA * wave + i)), a_live >> i & 1u);
  };
  auto issue_w = [&](int p) {  // pair p's weights into weight stage p % 2
    const uint8_t *wb = wbase + size_t(p) * 72;
    const uint32_t sw = lds0 + uint32_t(kW + (p & 1) * kP2WStage);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      dma<16>(wb, w_off[i], __builtin_amdgcn_readfirstlane(sw + uint32_t(wave * 4 * kW2Blk + i * kW2Blk)));
#pragma unroll
    for (int j = 0; j < 2; ++j)
      dma<4>(wb, d_off[j], __builtin_amdgcn_readfirstlane(sw + uint32_t(kW2X4) + 256u * uint32_t(2 * wave + j)));
  };

  f32x4 acc[4][MB];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const Q0Lane2 ql = q0_lane2<MODE>(wave, fr, g, 0);
  // step kk = 4 b + J: A stage J % 2, weight stage J / 2, unit J % 2 of the pair (compile-time LDS offsets)
  auto compute = [&](auto jj, auto qn) {
    constexpr int J = decltype(jj)::value, QN = decltype(qn)::value;
    q0_step_pair<QN, MB, J % 2>(lds + (J % 2) * kAStage, lds + kW + (J / 2) * kP2WStage, ql, fr, g, acc);
  };

  // Before step kk + 1 every wavefront waits for its copies of A(kk + 1), issued at the start of step kk, and of
  // the weights of pair (kk + 1) / 2, issued at step kk - 1 or earlier. The counter counts in issue order: on even
  // kk the 6 copies of pair kk / 2 + 1 went out after A(kk + 1) and may stay out; on odd kk nothing did.
  issue_a(0);
  issue_w(0);
  wait_vm<0>();
  barrier_lds();
  auto run = [&](auto qn) {
    for (int kb = 0; kb < nk; kb += 4) {
      static_for<0, 4>([&](auto j) {
        constexpr int J = decltype(j)::value;
        const int kk = kb + J;
        if (kk < nk) {
          if (kk + 1 < nk) issue_a(kk + 1);
          const bool w_out = J % 2 == 0 && kk / 2 + 1 < np;
          if (w_out) issue_w(kk / 2 + 1);
          compute(j, qn);
          if (kk + 1 < nk) {
            if (w_out)
              wait_vm<6>();
            else
              wait_vm<0>();
            barrier_lds();
          }
        }
      });
    }
  };
  if constexpr (QMAX == 2) {
    if (t.rows <= 32)  // uniform across the workgroup
      run(IC<1>{});
    else
      run(IC<2>{});
  } else {
    switch ((t.rows + 31) / 32) {  // uniform across the workgroup
      case 1: run(IC<1>{}); break;
      case 2: run(IC<2>{}); break;
      case 3: run(IC<3>{}); break;
      default: run(IC<4>{}); break;
    }
  }
  store_tile<MODE, MB>(acc, t, wave, fr, g, out, ldo, odt);
}

// Finishes a split-K grouped GEMM: rows p < offsets[E] (the grouped rows of real experts), 4 features a thread:
// the ksplit slices of ws added in slice order, then gate/up: h[p][K order of i] = f16(silu(g) u) for features
// i .. i + 3 of I; down: y[p][n] (F16 / F32). Grid (ceil(N / 1024), R): N = I (gate/up) or H (down).
template <int MODE>
__global__ void __launch_bounds__(256) k_splitk_finish(const float *ws, int ksplit, int R, int ldw,
                                                       const uint32_t *offsets, int E, void *out, int ldo, int odt) {
  const int p = blockIdx.y;
  if (p >= int(offsets[E])) return;
  const int n = (blockIdx.x * 256 + threadIdx.x) * 4;
  const int N = MODE == MODE_GATE_UP ? ldw / 2 : ldw;
  if (n >= N) return;
  f32x4 a = f32x4{0.0f, 0.0f, 0.0f, 0.0f}, b = a;
  for (int s = 0; s < ksplit; ++s) {
    const float *row = ws + (size_t(s) * R + p) * ldw;
    a += *reinterpret_cast<const f32x4 *>(row + n);
    if (MODE == MODE_GATE_UP) b += *reinterpret_cast<const f32x4 *>(row + N + n);
  }
  const size_t o = size_t(p) * ldo;
  if (MODE == MODE_GATE_UP) {
    const h2_t v01 = {_Float16(silu_mul_h(a[0], b[0])), _Float16(silu_mul_h(a[1], b[1]))};
    const h2_t v23 = {_Float16(silu_mul_h(a[2], b[2])), _Float16(silu_mul_h(a[3], b[3]))};
    *reinterpret_cast<u32x2 *>(static_cast<_Float16 *>(out) + o + kperm4(n)) =
        u32x2{__builtin_bit_cast(uint32_t, v01), __builtin_bit_cast(uint32_t, v23)};
  } else if (odt == LMOE_F32) {
    *reinterpret_cast<f32x4 *>(static_cast<float *>(out) + o + n) = a;
  } else {
    const h2_t v01 = {_Float16(a[0]), _Float16(a[1])}, v23 = {_Float16(a[2]), _Float16(a[3])};
    *reinterpret_cast<u32x2 *>(static_cast<_Float16 *>(out) + o + n) =
        u32x2{__builtin_bit_cast(uint32_t, v01), __builtin_bit_cast(uint32_t, v23)};
  }
}

// ---- f16 weights (the other block types, dequantized in the K order): both operands global -> LDS ---------------

constexpr int kFwDmaW = GN * 128 / 1024 / 4;         // 16-byte weight copies a lane a step (8)

// The grouped GEMMs over f16 weights [E][n_rows][K] already in the K order (lmoe_dequant_gemm_f16): the tiles,
// wavefront split, MFMA fragments and epilogue of k_grouped_q4_0, with the weight tile copied like the A tile
// (rows of 128 bytes, 16-byte chunks XOR-swizzled by the row's low 3 bits) and no decode. Two stages of a 32 KB
// weight tile plus the A tile: 128 rows (2 x 48 KB, one workgroup a CU) or 64 rows (2 x 40 KB, two a CU, each
// SIMD with two wavefronts to switch between). Step kk + 1's copies go out while step kk multiplies. Host
// guarantees: K % 64 == 0, rows x K x 2 of A and of one expert's weights under 4 GiB.
template <int MODE, int GMT = GM>
__global__ void __launch_bounds__(kThreads, GMT == 64 ? 2 : 1)
k_grouped_f16w(const _Float16 *a_src, int topk, const uint32_t *order, const uint32_t *offsets,
               const uint32_t *tiles, const uint32_t *n_tiles, int n_ntile, const _Float16 *w0, const _Float16 *w1,
               int K, int n_rows, void *out, int ldo, int odt) {
  constexpr int kFwAStage = GMT * 128, kFwStage = kFwAStage + GN * 128, kFwDmaA = GMT * 128 / 1024 / 4;
  constexpr int MB = GMT / 16, QMAX = GMT / 32;
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * kFwStage];
  Tile t;
  if (!tile_of<GMT>(offsets, tiles, n_tiles, n_ntile, &t)) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 15, g = lane >> 4;
  const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>(lds));

  // A as in k_grouped_q4_0: granule q = 64 (4 w + i) + lane holds chunk (q % 8) ^ (r & 7) of tile row r = q / 8
  uint32_t a_off[kFwDmaA];
#pragma unroll
  for (int i = 0; i < kFwDmaA; ++i) {
    const int q = 64 * (kFwDmaA * wave + i) + lane, r = q >> 3, c = (q & 7) ^ (r & 7);
    const int p = t.row0 + (r < t.rows ? r : 0);
    const uint32_t row = MODE == MODE_GATE_UP ? order[p] / uint32_t(topk) : uint32_t(p);
    a_off[i] = row * uint32_t(K) * 2u + 16u * uint32_t(c);
  }
  // weights: wavefront w covers tile features 64 w .. 64 w + 63 (gate/up: waves 0-1 gate rows, 2-3 up rows);
  // granule q = 64 (8 w + i) + lane holds chunk (q % 8) ^ (f & 7) of tile feature f = q / 8
  const _Float16 *wbase;
  uint32_t w_off[kFwDmaW];
  {
    const _Float16 *m = MODE == MODE_GATE_UP && wave >= 2 ? w1 : w0;
    const int row_base = MODE == MODE_GATE_UP ? t.nt * (GN / 2) - (wave >= 2 ? GN / 2 : 0) : t.nt * GN;
    wbase = m + size_t(t.e) * n_rows * K;
#pragma unroll
    for (int i = 0; i < kFwDmaW; ++i) {
      const int q = 64 * (kFwDmaW * wave + i) + lane, f = q >> 3, c = (q & 7) ^ (f & 7);
      w_off[i] = uint32_t(row_base + f) * uint32_t(K) * 2u + 16u * uint32_t(c);
    }
  }
  const int nk = K / GK;
  auto issue = [&](int kk) {  // step kk into stage kk % 2
    const uint32_t st = lds0 + uint32_t(kk & 1) * kFwStage;
    const _Float16 *ab = a_src + size_t(kk) * GK;
#pragma unroll
    for (int i = 0; i < kFwDmaA; ++i)
      dma<16>(ab, a_off[i], __builtin_amdgcn_readfirstlane(st + 1024u * uint32_t(kFwDmaA * wave + i)));
    const _Float16 *wb = wbase + size_t(kk) * GK;
#pragma unroll
    for (int i = 0; i < kFwDmaW; ++i)
      dma<16>(wb, w_off[i], __builtin_amdgcn_readfirstlane(st + kFwAStage + 1024u * uint32_t(kFwDmaW * wave + i)));
  };

  int wfeat[4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) wfeat[nb] = frag_feature<MODE>(wave, nb) + fr;
  f32x4 acc[4][MB];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  auto compute = [&](int s, auto qn) {
    constexpr int QN = decltype(qn)::value;
    const u32x4 *as = reinterpret_cast<const u32x4 *>(lds + s * kFwStage);
    const u32x4 *ws = reinterpret_cast<const u32x4 *>(lds + s * kFwStage + kFwAStage);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      half8 xf[8];
#pragma unroll
      for (int mb = 0; mb < 2 * QN; ++mb) xf[mb] = __builtin_bit_cast(half8, as[achunk(16 * mb + fr, 4 * ks + g)]);
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        const half8 wf = __builtin_bit_cast(half8, ws[achunk(wfeat[nb], 4 * ks + g)]);
#pragma unroll
        for (int mb = 0; mb < 2 * QN; ++mb)
          acc[nb][mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf, xf[mb], acc[nb][mb], 0, 0, 0);
      }
    }
  };

  // Step kk: step kk + 1's copies go out into the other stage (read in step kk - 1, released by its barrier),
  // step kk multiplies, then each wavefront waits for its own copies and the barrier publishes the stage.
  issue(0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  barrier_lds();
  auto run = [&](auto qn) {
    for (int kk = 0; kk < nk; ++kk) {
      if (kk + 1 < nk) issue(kk + 1);
      compute(kk & 1, qn);
      if (kk + 1 < nk) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        barrier_lds();
      }
    }
  };
  if constexpr (QMAX == 2) {
    if (t.rows <= 32)  // uniform across the workgroup
      run(IC<1>{});
    else
      run(IC<2>{});
  } else {
    switch ((t.rows + 31) / 32) {  // uniform across the workgroup
      case 1: run(IC<1>{}); break;
      case 2: run(IC<2>{}); break;
      case 3: run(IC<3>{}); break;
      default: run(IC<4>{}); break;
    }
  }
  store_tile<MODE, MB>(acc, t, wave, fr, g, out, ldo, odt);
}

// ---- Q4_K: register staging with repack --------------------------------------------------------------------------

constexpr int kWp = 10;  // LDS words a weight row a step: 8 nibble words, 2 scale words

// The super-block header (d, dmin, 12 scale bytes) and the 8 qs words of sub-block pair kk % 4 of a row
__device__ __forceinline__ void load_w_q4_k(const uint8_t *wrow, int kk, uint32_t *r) {
  const uint32_t *sb = reinterpret_cast<const uint32_t *>(wrow + size_t(kk >> 2) * 144);
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = sb[i];
#pragma unroll
  for (int i = 0; i < 8; ++i) r[4 + i] = sb[4 + 8 * (kk & 3) + i];
}

// o[4 ks + g]: slice ks = sub-block 2 (kk % 4) + ks (the low / high nibbles of the pair's 32 bytes); lane group g
// takes bytes 4g..4g+3 (low nibbles of the word) and 16 + 4g.. (high nibbles). o[8 + ks] = {f16(d sc), f16(dmin m)}
// of that sub-block (get_scale_min_k4, gguf_ref.py:253-258).
__device__ __forceinline__ void pack_w_q4_k(const uint32_t *r, int kk, uint32_t *o) {
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const uint32_t a = r[4 + g], b = r[8 + g];
    o[g] = (a & 0x0F0F0F0Fu) | ((b & 0x0F0F0F0Fu) << 4);
    o[4 + g] = ((a >> 4) & 0x0F0F0F0Fu) | (b & 0xF0F0F0F0u);
  }
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    float sc, mn;
    k4_scale_min(r[1], r[2], r[3], 2 * (kk & 3) + ks, &sc, &mn);
    const h2_t v = {_Float16(half_lo(r[0]) * sc), _Float16(half_hi(r[0]) * mn)};
    o[8 + ks] = __builtin_bit_cast(uint32_t, v);
  }
}

// Same grid and arguments as k_grouped_q4_0. GMT: tile rows (128, 64 or 32 for groups of fewer rows); D: K steps
// held in registers ahead of the one being staged (1 at 128 rows, where the accumulators leave no room; 2 at 64
// rows; 3 at 32 rows, so a step's loads have three steps of compute to arrive in).
template <int MODE, int GMT = GM, int D = 1>
__global__ void __launch_bounds__(kThreads, 2)
k_grouped_q4_k(const _Float16 *a_src, int topk, const uint32_t *order, const uint32_t *offsets,
               const uint32_t *tiles, const uint32_t *n_tiles, int n_ntile, const uint8_t *w0, const uint8_t *w1,
               int K, int n_rows, void *out, int ldo, int odt) {
  constexpr int MB = GMT / 16, QMAX = GMT / 32, AQ = GMT * 8 / kThreads;  // A granules a thread a step
  static_assert(AQ >= 1 && D >= 1 && D <= 3, "tile and prefetch shape");
  // A tile: rows of 64 halves = 8 swizzled 16-byte chunks; packed weights: kWp words a tile feature; 2 stages each
  __shared__ __attribute__((aligned(16))) u32x4 As[2][GMT * 8];
  __shared__ __attribute__((aligned(16))) uint32_t Wp[2][GN * kWp];
  Tile t;
  if (!tile_of<GMT>(offsets, tiles, n_tiles, n_ntile, &t)) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fr = lane & 15, g = lane >> 4;
  const size_t wrow_bytes = size_t(144) * (K / 256);

  // A staging: thread -> tile row ar = tid / (256 / GMT), its AQ contiguous 16-byte chunks from c0 (128 rows: 2
  // threads a row, 4 chunks each; 32 rows: 8 threads a row, 1 chunk each). Rows past the tile's end read the tile's
  // first row instead (their results are never stored).
  constexpr int TPR = kThreads / GMT;
  const int ar = tid / TPR, c0 = (tid % TPR) * AQ;
  const u32x4 *a_ptr;
  {
    const int p = t.row0 + (ar < t.rows ? ar : 0);
    const size_t r = MODE == MODE_GATE_UP ? size_t(order[p] / uint32_t(topk)) : size_t(p);
    a_ptr = reinterpret_cast<const u32x4 *>(a_src + r * K) + c0;
  }
  // weight staging: thread -> tile feature tid
  const uint8_t *w_row;
  if (MODE == MODE_GATE_UP)
    w_row = (tid < GN / 2 ? w0 : w1) + (size_t(t.e) * n_rows + t.nt * (GN / 2) + (tid % (GN / 2))) * wrow_bytes;
  else
    w_row = w0 + (size_t(t.e) * n_rows + t.nt * GN + tid) * wrow_bytes;

  int wfeat[4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) wfeat[nb] = frag_feature<MODE>(wave, nb) + fr;

  u32x4 areg[D][AQ];
  uint32_t wraw[D][12];
  f32x4 acc[4][MB];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  auto load = [&](int kk, auto slot) {  // raw weights and A of step kk into register slot `slot`
    constexpr int S = decltype(slot)::value;
    load_w_q4_k(w_row, kk, wraw[S]);
#pragma unroll
    for (int i = 0; i < AQ; ++i) areg[S][i] = a_ptr[size_t(kk) * (GK / 8) + i];
  };
  auto stage = [&](int l, int kk, auto slot) {  // register slot -> LDS stage l
    constexpr int S = decltype(slot)::value;
#pragma unroll
    for (int i = 0; i < AQ; ++i) As[l][achunk(ar, c0 + i)] = areg[S][i];
    uint32_t o[kWp];
    pack_w_q4_k(wraw[S], kk, o);
#pragma unroll
    for (int j = 0; j < kWp; ++j) Wp[l][tid * kWp + j] = o[j];
  };
  // 64 MFMAs out of LDS stage l: per K slice, the 4 weight fragments are decoded from their packed words, then
  // each A fragment meets all 4
  auto compute = [&](int l, auto qn) {  // qn: the 32-row pairs the tile has rows in, as in the Q4_0 kernel
    constexpr int QN = decltype(qn)::value;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      half8 wf[4];
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
        wf[nb] = decode8<LMOE_Q4_K>(Wp[l][wfeat[nb] * kWp + 4 * ks + g], Wp[l][wfeat[nb] * kWp + 8 + ks], 0);
#pragma unroll
      for (int mb = 0; mb < 2 * QN; ++mb) {
        const half8 xf = __builtin_bit_cast(half8, As[l][achunk(16 * mb + fr, 4 * ks + g)]);
#pragma unroll
        for (int nb = 0; nb < 4; ++nb)
          acc[nb][mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[nb], xf, acc[nb][mb], 0, 0, 0);
      }
    }
  };
  // Step kk: issue the global loads of step kk + D into the register slot step kk left (staged one step ago),
  // multiply out of LDS stage kk % 2 (the loads are in flight meanwhile), then stage step kk + 1 from its slot
  // into the other LDS stage; one barrier a step. Register slots are compile-time indices, so the loop is written
  // D steps at a time.
  const int nk = K / GK;
  load(0, IC<0>{});
  if (D > 1 && nk > 1) load(1, IC<(D > 1 ? 1 : 0)>{});
  if (D > 2 && nk > 2) load(2, IC<(D > 2 ? 2 : 0)>{});
  stage(0, 0, IC<0>{});
  __syncthreads();
  auto run = [&](auto qn) {
    if constexpr (D == 1) {  // one slot: the last step's multiply outside the loop, no branch inside it
      for (int kk = 0; kk + 1 < nk; ++kk) {
        load(kk + 1, IC<0>{});
        __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of the MFMAs
        compute(kk & 1, qn);
        stage((kk + 1) & 1, kk + 1, IC<0>{});
        __syncthreads();
      }
      compute((nk - 1) & 1, qn);
      return;
    }
    auto step = [&](int kk, auto j) {  // j = kk % D
      constexpr int J = decltype(j)::value, JN = (J + 1) % D;
      if (kk + D < nk) load(kk + D, IC<J>{});
      __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of the MFMAs (the scheduler sinks them otherwise)
      compute(kk & 1, qn);
      if (kk + 1 < nk) {
        stage((kk + 1) & 1, kk + 1, IC<JN>{});
        __syncthreads();
      }
    };
    for (int base = 0; base < nk; base += D) {
      step(base, IC<0>{});
      if (D > 1 && base + 1 < nk) step(base + 1, IC<(D > 1 ? 1 : 0)>{});
      if (D > 2 && base + 2 < nk) step(base + 2, IC<(D > 2 ? 2 : 0)>{});
    }
  };
  if constexpr (QMAX == 1) {
    run(IC<1>{});
  } else if constexpr (QMAX == 2) {
    if (t.rows <= 32)  // uniform across the workgroup
      run(IC<1>{});
    else
      run(IC<2>{});
  } else {
    switch ((t.rows + 31) / 32) {  // uniform across the workgroup
      case 1: run(IC<1>{}); break;
      case 2: run(IC<2>{}); break;
      case 3: run(IC<3>{}); break;
      default: run(IC<4>{}); break;
    }
  }
  store_tile<MODE, MB>(acc, t, wave, fr, g, out, ldo, odt);
}

// ---- Q4_K: global -> LDS directly, four stages of 64-row tiles --------------------------------------------------

// LDS: NST stages of the A tile (GMT rows x 64 K, f16, swizzled rows of 128 bytes as in the Q4_0 kernel) and the
// step's 32 qs bytes of every tile feature (two 16-byte halves: each group of 16 features keeps its first halves in
// one 256-byte row and its second halves in the next, as the Q4_0 unit heads); one buffer of super-block headers
// (d, dmin, 12 scale bytes: 16 bytes a feature), copied with the first step of each super-block; and the table of
// the current super-block's 8 (f16(d sc), f16(dmin m)) pairs of every feature, 40 bytes a feature so that the 16
// features of an MFMA fragment read 16 different bank pairs.
constexpr int kKQs = GN * 32, kKHd = GN * 16, kKTabRow = 40, kKTab = GN * kKTabRow;
template <int GMT> constexpr int qk_astage() { return GMT * 128; }
template <int GMT> constexpr int qk_stage() { return qk_astage<GMT>() + kKQs; }

// The Q4_K grouped GEMMs on the copy ring of k_grouped_q4_0: A and the step's raw qs bytes go global -> LDS directly
// (global_load_lds, no registers), NST - 1 K steps ahead, one barrier a step; each super-block's header goes with
// its first step. When a super-block starts, thread t turns feature t's header into the table of its 8 sub-block
// scale pairs (get_scale_min_k4, gguf_ref.py:253-258; one more barrier every 4 steps). Each MFMA lane then builds
// its nibble word from qs words g and g + 4 of its feature (the low nibbles for the step's first sub-block, the
// high nibbles for its second: ggml's Q4_K packs sub-blocks 2s and 2s + 1 of pair s in one 32-byte run) and
// decodes it with its pair from the table. 64-row tiles: a 16 KB stage, four stages, two workgroups a CU, three
// steps in flight: streaming a different expert's weights through every tile (prefill over many experts with few
// rows each). Grid and arguments as k_grouped_q4_0; host guarantees: K % 256 == 0, rows x K x 2 of A and one
// expert's weight block under 4 GiB.
template <int MODE, int GMT = 64, int NST = 4, bool SL = false>
__global__ void __launch_bounds__(kThreads, 2)
k_grouped_q4_k_dma(const _Float16 *a_src, int topk, const uint32_t *order, const uint32_t *offsets,
                   const uint32_t *tiles, const uint32_t *n_tiles, int n_ntile, const uint8_t *w0, const uint8_t *w1,
                   int K, int n_rows, void *out, int ldo, int odt) {
  constexpr int kAStage = qk_astage<GMT>(), kStage = qk_stage<GMT>(), kDmaA = GMT * 128 / 1024 / 4;
  constexpr int kHd = NST * kStage, kTab = kHd + kKHd;
  constexpr int MB = GMT / 16, QMAX = GMT / 32;
  static_assert(kDmaA >= 1 && NST >= 3 && kTab + kKTab <= 81920, "tile and pipeline shape");
  __shared__ __attribute__((aligned(16))) uint8_t lds[kTab + kKTab];
  Tile t;
  if (!tile_of<GMT>(offsets, tiles, n_tiles, n_ntile, &t)) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 15, g = lane >> 4;
  const uint32_t wrow = 144u * uint32_t(K / 256);
  const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>(lds));

  // A: as in k_grouped_q4_0
  uint32_t a_off[kDmaA];
#pragma unroll
  for (int i = 0; i < kDmaA; ++i) {
    const int q = 64 * (kDmaA * wave + i) + lane, r = q >> 3, c = (q & 7) ^ (r & 7);
    const int p = t.row0 + (r < t.rows ? r : 0);
    const uint32_t row = MODE == MODE_GATE_UP ? order[p] / uint32_t(topk) : uint32_t(p);
    a_off[i] = row * uint32_t(K) * 2u + 16u * uint32_t(c);
  }
  const uint32_t a_live = a_live_mask<kDmaA>(wave, t.rows);
  // weights: wavefront w copies tile features 64 w .. 64 w + 63 (gate/up: waves 0-1 gate rows, 2-3 up rows).
  // qs copy i: granule q = 64 (2 w + i) + lane is half h = (q / 16) % 2 of feature f = 16 (q / 32) + q % 16, from
  // super-block byte 16 + 16 h (+ 32 s of step pair s). Header copy: feature 64 w + lane's first 16 bytes.
  const uint8_t *wbase;
  uint32_t q_off[2], h_off;
  if constexpr (SL) {
    // the stream layout (k_stream_repack): wavefront w's 128-feature block fb, one 18,432-byte block a super-block
    // (the headers, then the 4 steps' qs): each copy reads one contiguous kilobyte
    const uint8_t *m = MODE == MODE_GATE_UP && wave >= 2 ? w1 : w0;
    const int fb = MODE == MODE_GATE_UP ? t.nt : 2 * t.nt + (wave >> 1);
    wbase = m + (size_t(t.e) * (n_rows / 128) + fb) * size_t(K / 256) * kSlQK;
#pragma unroll
    for (int i = 0; i < 2; ++i) q_off[i] = 2048u + 16u * uint32_t(64 * (2 * (wave & 1) + i) + lane);
    h_off = 16u * uint32_t(64 * (wave & 1) + lane);
  } else {
    const uint8_t *m = MODE == MODE_GATE_UP && wave >= 2 ? w1 : w0;
    const int row_base = MODE == MODE_GATE_UP ? t.nt * (GN / 2) - (wave >= 2 ? GN / 2 : 0) : t.nt * GN;
    wbase = m + (size_t(t.e) * n_rows) * wrow;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int q = 64 * (2 * wave + i) + lane;
      q_off[i] = uint32_t(row_base + 16 * (q >> 5) + (q & 15)) * wrow + 16u + 16u * uint32_t((q >> 4) & 1);
    }
    h_off = uint32_t(row_base + 64 * wave + lane) * wrow;
  }
  const int nk = K / GK;
  auto issue = [&](int kk) {  // step kk into stage kk % NST (its super-block's header too when kk % 4 == 0)
    const uint32_t st = lds0 + uint32_t(kk % NST) * kStage;
    const _Float16 *ab = a_src + size_t(kk) * GK;
#pragma unroll
    for (int i = 0; i < kDmaA; ++i)
      dma_a(ab, a_off[i], __builtin_amdgcn_readfirstlane(st + 1024u * uint32_t(kDmaA * wave + i)), a_live >> i & 1u);
    const uint8_t *sb = wbase + size_t(kk >> 2) * (SL ? kSlQK : 144);
    const uint8_t *qb = sb + (SL ? 4096 : 32) * (kk & 3);
#pragma unroll
    for (int i = 0; i < 2; ++i)
      dma<16>(qb, q_off[i], __builtin_amdgcn_readfirstlane(st + kAStage + 1024u * uint32_t(2 * wave + i)));
    if ((kk & 3) == 0) dma<16>(sb, h_off, __builtin_amdgcn_readfirstlane(lds0 + kHd + 1024u * uint32_t(wave)));
  };
  // the scale pairs of feature tid's current super-block, from its header: table row tid, pair j at 4 j
  auto fill_table = [&] {
    const u32x4 h = *reinterpret_cast<const u32x4 *>(lds + kHd + 16 * tid);
    const uint32_t h0 = h[0], h1 = h[1], h2 = h[2], h3 = h[3];
    const float d = half_lo(h0), dmin = half_hi(h0);
    uint32_t v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float sc, mn;
      k4_scale_min(h1, h2, h3, j, &sc, &mn);
      v[j] = __builtin_bit_cast(uint32_t, h2_t{_Float16(d * sc), _Float16(dmin * mn)});
    }
    uint32_t *row = reinterpret_cast<uint32_t *>(lds + kTab + kKTabRow * tid);
#pragma unroll
    for (int j = 0; j < 8; j += 2) *reinterpret_cast<u32x2 *>(row + j) = u32x2{v[j], v[j + 1]};
  };

  f32x4 acc[4][MB];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  // lane (fr, g) of fragment nb: feature f = frag_feature(nb) + fr; its qs words g and g + 4 sit at qlo[nb] and
  // qlo[nb] + 256 of a stage, its scale pairs in table row f
  int qlo[4], tab[4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) {
    const int f = frag_feature<MODE>(wave, nb) + fr;
    qlo[nb] = kAStage + 512 * (f >> 4) + 16 * (f & 15) + 4 * g;
    tab[nb] = kTab + kKTabRow * f;
  }
  // Step kk out of stage s: per fragment the two qs words and the step's two scale pairs, both K slices' weights
  // decoded, each meeting the tile's A fragments (NMB 16-row blocks: a 40-row group multiplies 48 rows, not 64)
  auto compute = [&](auto s, int kk, auto nmb) {  // s: the stage, a compile-time index (immediate LDS offsets)
    constexpr int NMB = decltype(nmb)::value;
    const uint8_t *st = lds + decltype(s)::value * kStage;
    const u32x4 *as = reinterpret_cast<const u32x4 *>(st);
    const int pr = kk & 3;  // the step's sub-block pair: sub-blocks 2 pr (low nibbles) and 2 pr + 1 (high)
    half8 xf[2][MB];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb) xf[ks][mb] = __builtin_bit_cast(half8, as[achunk(16 * mb + fr, 4 * ks + g)]);
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      const uint32_t lo = *reinterpret_cast<const uint32_t *>(st + qlo[nb]);
      const uint32_t hi = *reinterpret_cast<const uint32_t *>(st + qlo[nb] + 256);
      const u32x2 sp = *reinterpret_cast<const u32x2 *>(lds + tab[nb] + 8 * pr);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const uint32_t x = ks == 0 ? (lo & 0x0F0F0F0Fu) | ((hi & 0x0F0F0F0Fu) << 4)
                                   : ((lo >> 4) & 0x0F0F0F0Fu) | (hi & 0xF0F0F0F0u);
        const half8 wf = decode8<LMOE_Q4_K>(x, ks == 0 ? uint32_t(sp[0]) : uint32_t(sp[1]), 0);
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb)
          acc[nb][mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf, xf[ks][mb], acc[nb][mb], 0, 0, 0);
      }
    }
  };

  // the ring of k_grouped_q4_0: step kk + NST - 1's copies go out, step kk multiplies, each wavefront waits for its
  // own copies of step kk + 1 and the barrier publishes that stage (and frees stage kk for the refill after it).
  // A step makes C copies a lane, C + 1 when it starts a super-block; the waits count C a step, so they may also
  // wait for one copy of the step after (never less than they must).
  constexpr int C = kDmaA + 2;
  static_assert(NST <= 5 && 3 * C + 3 <= 63, "the wait counts below");
  auto wait_steps = [&](int later) {
    if (later <= 0)
      wait_vm<0>();
    else if (later == 1)
      wait_vm<C>();
    else if (later == 2)
      wait_vm<2 * C>();
    else
      wait_vm<3 * C>();
  };
  const int pre = min(NST - 1, nk);
  for (int j = 0; j < pre; ++j) issue(j);
  wait_steps(pre - 1);
  barrier_lds();
  auto run = [&](auto qn) {
    for (int kb = 0; kb < nk; kb += NST) {  // NST steps a pass, so step kb + j reads stage j
      static_for<0, NST>([&](auto j) {
        const int kk = kb + decltype(j)::value;
        if (kk < nk) {
          if ((kk & 3) == 0) {  // the super-block's header landed with this step: its scale table, then a barrier
            fill_table();
            barrier_lds();
          }
          if (kk + NST - 1 < nk) issue(kk + NST - 1);
          compute(j, kk, qn);
          if (kk + 1 < nk) {
            wait_steps(min(kk + NST - 1, nk - 1) - (kk + 1));
            barrier_lds();
          }
        }
      });
    }
  };
  switch ((t.rows + 15) / 16) {  // uniform across the workgroup
    case 1: run(IC<1>{}); break;
    case 2: run(IC<(MB >= 2 ? 2 : MB)>{}); break;
    case 3: run(IC<(MB >= 3 ? 3 : MB)>{}); break;
    default: run(IC<MB>{}); break;
  }
  store_tile<MODE, MB>(acc, t, wave, fr, g, out, ldo, odt);
}

// k_grouped_q4_k_dma<MODE, 64> on the GGUF layout with the weights staged two steps at a time. A one-step stage
// copies 32 qs bytes of each of 256 weight rows (a 128-byte line a row for 32 of its bytes) and the line has left
// L1 before the next step wants its neighbour; a step pair's 64 qs bytes are contiguous (runs 2j, 2j + 1 of a
// super-block). LDS: four one-step A stages (three steps ahead, 8 KB each), two pair stages of weights (one pair
// ahead: wavefront w's rows as 4 blocks of 16 rows x 64 bytes padded to 1,040 bytes, feature 16 q + 4 i + j at
// block i slot 4 q + j, so an MFMA fragment's 16 features sit in 16 different 4-bank groups), the header buffer
// and the scale table of k_grouped_q4_k_dma. Arithmetic and order as k_grouped_q4_k_dma<MODE, 64, 4>: the same
// bits. Grid, arguments and host guarantees as there.
constexpr int kKW2Stage = 4 * 4 * kW2Blk;  // a pair stage: 4 wavefronts x 4 blocks
template <int MODE>
__global__ void __launch_bounds__(kThreads, 2)
k_grouped_q4_k_w2(const _Float16 *a_src, int topk, const uint32_t *order, const uint32_t *offsets,
                  const uint32_t *tiles, const uint32_t *n_tiles, int n_ntile, const uint8_t *w0, const uint8_t *w1,
                  int K, int n_rows, void *out, int ldo, int odt) {
  constexpr int GMT = 64, NA = 4;
  constexpr int kAStage = qk_astage<GMT>(), kDmaA = GMT * 128 / 1024 / 4;
  constexpr int kW = NA * kAStage, kHd = kW + 2 * kKW2Stage, kTab = kHd + kKHd;
  constexpr int MB = GMT / 16;
  static_assert(kTab + kKTab <= 81920, "two workgroups a CU");
  __shared__ __attribute__((aligned(16))) uint8_t lds[kTab + kKTab];
  Tile t;
  if (!tile_of<GMT>(offsets, tiles, n_tiles, n_ntile, &t)) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 15, g = lane >> 4;
  const uint32_t wrow = 144u * uint32_t(K / 256);
  const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>(lds));

  uint32_t a_off[kDmaA];  // A: as in k_grouped_q4_0
#pragma unroll
  for (int i = 0; i < kDmaA; ++i) {
    const int q = 64 * (kDmaA * wave + i) + lane, r = q >> 3, c = (q & 7) ^ (r & 7);
    const int p = t.row0 + (r < t.rows ? r : 0);
    const uint32_t row = MODE == MODE_GATE_UP ? order[p] / uint32_t(topk) : uint32_t(p);
    a_off[i] = row * uint32_t(K) * 2u + 16u * uint32_t(c);
  }
  const uint32_t a_live = a_live_mask<kDmaA>(wave, t.rows);
  // weights: wavefront w copies tile features 64 w .. 64 w + 63 (gate/up: waves 0-1 gate rows, 2-3 up rows). Pair
  // copy i: lane l takes bytes 16 (l % 4) .. of the pair's 64 qs bytes of feature 16 (s / 4) + 4 i + s % 4,
  // s = l / 4. Header copy: feature 64 w + lane's first 16 bytes of the super-block.
  const uint8_t *m = MODE == MODE_GATE_UP && wave >= 2 ? w1 : w0;
  const int row_base = (MODE == MODE_GATE_UP ? t.nt * (GN / 2) - (wave >= 2 ? GN / 2 : 0) : t.nt * GN) + 64 * wave;
  const uint8_t *wbase = m + (size_t(t.e) * n_rows) * wrow;
  uint32_t q_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int s = lane >> 2, fl = 16 * (s >> 2) + 4 * i + (s & 3);
    q_off[i] = uint32_t(row_base + fl) * wrow + 16u + 16u * uint32_t(lane & 3);
  }
  const uint32_t h_off = uint32_t(row_base + lane) * wrow;
  const int nk = K / GK, np = nk / 2;
  auto issue_a = [&](int kk) {  // step kk's A into A stage kk % NA
    const uint32_t st = lds0 + uint32_t(kk % NA) * kAStage;
    const _Float16 *ab = a_src + size_t(kk) * GK;
#pragma unroll
    for (int i = 0; i < kDmaA; ++i)
      dma_a(ab, a_off[i], __builtin_amdgcn_readfirstlane(st + 1024u * uint32_t(kDmaA * wave + i)), a_live >> i & 1u);
  };
  auto issue_w = [&](int p) {  // pair p's qs into pair stage p % 2, then its super-block's header when p is even
    const uint8_t *sb = wbase + size_t(p >> 1) * 144;
    const uint8_t *qb = sb + 64 * (p & 1);
    const uint32_t sw = lds0 + uint32_t(kW + (p & 1) * kKW2Stage + wave * 4 * kW2Blk);
#pragma unroll
    for (int i = 0; i < 4; ++i) dma<16>(qb, q_off[i], __builtin_amdgcn_readfirstlane(sw + uint32_t(i * kW2Blk)));
    if ((p & 1) == 0) dma<16>(sb, h_off, __builtin_amdgcn_readfirstlane(lds0 + kHd + 1024u * uint32_t(wave)));
  };
  auto fill_table = [&] {  // as in k_grouped_q4_k_dma
    const u32x4 h = *reinterpret_cast<const u32x4 *>(lds + kHd + 16 * tid);
    const uint32_t h0 = h[0], h1 = h[1], h2 = h[2], h3 = h[3];
    const float d = half_lo(h0), dmin = half_hi(h0);
    uint32_t v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float sc, mn;
      k4_scale_min(h1, h2, h3, j, &sc, &mn);
      v[j] = __builtin_bit_cast(uint32_t, h2_t{_Float16(d * sc), _Float16(dmin * mn)});
    }
    uint32_t *row = reinterpret_cast<uint32_t *>(lds + kTab + kKTabRow * tid);
#pragma unroll
    for (int j = 0; j < 8; j += 2) *reinterpret_cast<u32x2 *>(row + j) = u32x2{v[j], v[j + 1]};
  };

  f32x4 acc[4][MB];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  // lane (fr, g) of fragment nb: feature f = frag_feature(nb) + fr; its qs words g and g + 4 of run u of the pair
  // at qx[nb] + 32 u and qx[nb] + 32 u + 16 of a pair stage, its scale pairs in table row f
  int qx[4], tab[4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) {
    const int f = frag_feature<MODE>(wave, nb) + fr;
    const int cw = f >> 6, fl = f & 63, q = fl >> 4, i = (fl >> 2) & 3, j = fl & 3;
    qx[nb] = kW + cw * 4 * kW2Blk + i * kW2Blk + 64 * (4 * q + j) + 4 * g;
    tab[nb] = kTab + kKTabRow * f;
  }
  // step kk = 4 b + J: A stage J, pair stage J / 2, run J % 2 of the pair, sub-block pair J of the super-block
  auto compute = [&](auto jj, auto nmb) {
    constexpr int J = decltype(jj)::value, NMB = decltype(nmb)::value;
    const u32x4 *as = reinterpret_cast<const u32x4 *>(lds + J * kAStage);
    const uint8_t *sq = lds + (J / 2) * kKW2Stage + 32 * (J % 2);
    half8 xf[2][MB];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb) xf[ks][mb] = __builtin_bit_cast(half8, as[achunk(16 * mb + fr, 4 * ks + g)]);
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      const uint32_t lo = *reinterpret_cast<const uint32_t *>(sq + qx[nb]);
      const uint32_t hi = *reinterpret_cast<const uint32_t *>(sq + qx[nb] + 16);
      const u32x2 sp = *reinterpret_cast<const u32x2 *>(lds + tab[nb] + 8 * J);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const uint32_t x = ks == 0 ? (lo & 0x0F0F0F0Fu) | ((hi & 0x0F0F0F0Fu) << 4)
                                   : ((lo >> 4) & 0x0F0F0F0Fu) | (hi & 0xF0F0F0F0u);
        const half8 wf = decode8<LMOE_Q4_K>(x, ks == 0 ? uint32_t(sp[0]) : uint32_t(sp[1]), 0);
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb)
          acc[nb][mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf, xf[ks][mb], acc[nb][mb], 0, 0, 0);
      }
    }
  };

  // Step kk: A of step kk + 3 goes out, and on even kk the weights of pair kk / 2 + 1 (the pair stage that pair
  // kk / 2 - 1 left); step kk multiplies; then each wavefront waits for its own copies of step kk + 1 and the
  // barrier publishes them. The counter counts in issue order. Copies a lane: CA a step, 4 a pair, 1 a header.
  // Before step kk + 1 (odd kk) the last copies that may still be out are A of step kk + 3 (CA); before step
  // kk + 1 (even kk) those of steps kk + 2 and kk + 3 and pair kk / 2 + 1 (2 CA + 4, or one more with a header:
  // waiting for 2 CA + 4 then also waits for one later copy, never too little). With fewer than 3 steps left
  // nothing is counted: the wait is for every copy.
  constexpr int CA = kDmaA;
  static_assert(2 * CA + 5 <= 63, "the wait counts below");
  issue_a(0);
  issue_a(1);
  issue_w(0);
  if (nk > 2) issue_a(2);
  wait_vm<0>();
  barrier_lds();
  auto run = [&](auto nmb) {
    for (int kb = 0; kb < nk; kb += 4) {  // K % 256 == 0: whole super-blocks, four steps a pass
      static_for<0, 4>([&](auto j) {
        constexpr int J = decltype(j)::value;
        const int kk = kb + J;
        if constexpr (J == 0) {  // the super-block's header landed with its first pair: its scale table
          fill_table();
          barrier_lds();
        }
        if (kk + 3 < nk) issue_a(kk + 3);
        if (J % 2 == 0 && kk / 2 + 1 < np) issue_w(kk / 2 + 1);
        compute(j, nmb);
        if (kk + 1 < nk) {
          if (kk + 3 >= nk)
            wait_vm<0>();
          else if (J % 2 == 1)
            wait_vm<CA>();
          else
            wait_vm<2 * CA + 4>();
          barrier_lds();
        }
      });
    }
  };
  switch ((t.rows + 15) / 16) {  // uniform across the workgroup
    case 1: run(IC<1>{}); break;
    case 2: run(IC<2>{}); break;
    case 3: run(IC<3>{}); break;
    default: run(IC<MB>{}); break;
  }
  store_tile<MODE, MB>(acc, t, wave, fr, g, out, ldo, odt);
}

// x [n] in dt -> f16 (round to nearest even), 8 elements a thread (vector loads when the whole range allows).
// kperm: element i lands at its position in the grouped GEMMs' K order (n % 32 == 0, vector path only).
__global__ void __launch_bounds__(256) k_to_f16(const void *x, int dt, long long n, _Float16 *out, int vec,
                                                int kperm) {
  if (vec && kperm) {
    to_f16_kperm(blockIdx.x, x, dt, n, out);
    return;
  }
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

// ---- the prefill router: logits = x . wr^T on the matrix cores ------------------------------------------------

constexpr int kRgM = 64, kRgN = 128;  // tokens and logit rows a tile
constexpr int kRgAStage = kRgM * 128, kRgStage = kRgAStage + kRgN * 128, kRgNst = 3;

// Router logits for a prefill chunk: x [T][K] and w [E + n_gate][K] both f16 in the grouped GEMMs' K order (the
// x the experts read, and the router weight converted once), fp32 accumulation of exact f16 products. A tile is
// 64 tokens x 128 logit rows, four wavefronts of 64 tokens x 32 rows (2 x 4 accumulators of
// v_mfma_f32_16x16x32_f16, the weight rows as the first operand); both operands go global -> LDS directly, three
// stages, as in the grouped GEMMs. ksplit > 1: workgroup kpart takes K steps [kpart nk, (kpart + 1) nk) and writes
// its sums to part[kpart][t][ldp] (k_router_finish adds the slices in slice order); ksplit == 1: logits straight
// out. Rows past T read token T - 1 and logit rows past E read row E - 1; neither is stored. Logit row E (the
// shared expert's gate, n_gate == 1) goes to gate[t].
__global__ void __launch_bounds__(kThreads, 2)
k_router_gemm(const _Float16 *x, int T, const _Float16 *w, int En, int K, int n_ntile, int ksplit, float *part,
              int ldp, float *logits, int E, float *gate) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kRgNst * kRgStage];
  const int b = blockIdx.x;
  const int kpart = b % ksplit, tile = b / ksplit;
  const int nt = tile % n_ntile, mt = tile / n_ntile;
  const int row0 = mt * kRgM, col0 = nt * kRgN;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 15, g = lane >> 4;
  const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>(lds));
  // x: copy i carries granule q = 64 (2 w + i) + lane = chunk (q % 8) ^ (r % 8) of token row r = q / 8;
  // w: copy i carries granule q = 64 (4 w + i) + lane of logit row f = q / 8
  uint32_t a_off[2], w_off[4];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int q = 64 * (2 * wave + i) + lane, r = q >> 3, c = (q & 7) ^ (r & 7);
    a_off[i] = uint32_t(min(row0 + r, T - 1)) * uint32_t(K) * 2u + 16u * uint32_t(c);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int q = 64 * (4 * wave + i) + lane, f = q >> 3, c = (q & 7) ^ (f & 7);
    w_off[i] = uint32_t(min(col0 + f, En - 1)) * uint32_t(K) * 2u + 16u * uint32_t(c);
  }
  const int nk = K / GK / ksplit, k0 = kpart * nk;
  auto issue = [&](int kk) {
    const uint32_t st = lds0 + uint32_t(kk % kRgNst) * kRgStage;
    const _Float16 *ab = x + size_t(k0 + kk) * GK;
#pragma unroll
    for (int i = 0; i < 2; ++i)
      dma<16>(ab, a_off[i], __builtin_amdgcn_readfirstlane(st + 1024u * uint32_t(2 * wave + i)));
    const _Float16 *wb = w + size_t(k0 + kk) * GK;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      dma<16>(wb, w_off[i], __builtin_amdgcn_readfirstlane(st + kRgAStage + 1024u * uint32_t(4 * wave + i)));
  };
  f32x4 acc[2][4];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb)
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) acc[nb][mb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  auto compute = [&](int s) {
    const u32x4 *as = reinterpret_cast<const u32x4 *>(lds + s * kRgStage);
    const u32x4 *ws = reinterpret_cast<const u32x4 *>(lds + s * kRgStage + kRgAStage);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      half8 xf[4];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) xf[mb] = __builtin_bit_cast(half8, as[achunk(16 * mb + fr, 4 * ks + g)]);
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const half8 wf = __builtin_bit_cast(half8, ws[achunk(32 * wave + 16 * nb + fr, 4 * ks + g)]);
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
          acc[nb][mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf, xf[mb], acc[nb][mb], 0, 0, 0);
      }
    }
  };
  constexpr int C = 6;  // copies a lane a step
  issue(0);
  if (nk > 1) issue(1);
  if (nk > 1)
    wait_vm<C>();
  else
    wait_vm<0>();
  barrier_lds();
  for (int kk = 0; kk < nk; ++kk) {
    if (kk + 2 < nk) issue(kk + 2);
    compute(kk % kRgNst);
    if (kk + 1 < nk) {
      if (kk + 2 < nk)
        wait_vm<C>();
      else
        wait_vm<0>();
      barrier_lds();
    }
  }
  // acc[nb][mb][r] = sum over this slice for logit row col0 + 32 w + 16 nb + 4 g + r, token row0 + 16 mb + fr
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    const int t = row0 + 16 * mb + fr;
    if (t >= T) continue;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int e = col0 + 32 * wave + 16 * nb + 4 * g;
      if (ksplit > 1) {
        *reinterpret_cast<f32x4 *>(part + (size_t(kpart) * T + t) * ldp + e) = acc[nb][mb];
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (e + r < E)
            logits[size_t(t) * E + e + r] = acc[nb][mb][r];
          else if (e + r < En)
            gate[t] = acc[nb][mb][r];
        }
      }
    }
  }
}

// Adds the ksplit slices of k_router_gemm in slice order: logits[t][e] (e < E), gate[t] (e == E < En).
// Grid (ceil(En / 256), T).
__global__ void __launch_bounds__(256) k_router_finish(const float *part, int ksplit, int T, int ldp, int En, int E,
                                                       float *logits, float *gate) {
  const int t = blockIdx.y, e = blockIdx.x * 256 + threadIdx.x;
  if (e >= En) return;
  float v = 0.0f;
  for (int s = 0; s < ksplit; ++s) v += part[(size_t(s) * T + t) * ldp + e];
  if (e < E)
    logits[size_t(t) * E + e] = v;
  else
    gate[t] = v;
}

// The split-K finish and the top-k in one launch, four tokens a workgroup, one wavefront each: each logit is its
// slices added in slice order from zero (k_router_finish's sums, written to logits / gate as it would), then
// topk_wave; with m > 0 slots k .. k + m - 1 are the folded shared expert's slices (E + j, sigmoid(gate logit)), as
// in k_router_topk.
// KS: the K split (2, 4 or 8), so that every slice's loads go out before the first add.
template <int NPL, int KS>
__global__ void __launch_bounds__(256) k_topk_from_parts(const float *part, int T, int ldp, int E, int n_gate, int k,
                                                         int norm, int m, float *logits, float *gate, uint32_t *ids,
                                                         float *scores) {
  __shared__ __attribute__((aligned(16))) uint32_t scr[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;
  float p[KS][NPL], pg[KS];
#pragma unroll
  for (int q = 0; q < KS; ++q) {
    const float *row = part + (size_t(q) * T + t) * ldp;
#pragma unroll
    for (int j = 0; j < NPL; ++j) p[q][j] = row[min(lane + 64 * j, E - 1)];
    pg[q] = row[n_gate ? E : 0];
  }
  float v[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    float a = 0.0f;
#pragma unroll
    for (int q = 0; q < KS; ++q) a += p[q][j];  // slice order, from zero: k_router_finish's sum
    if (lane + 64 * j < E) logits[size_t(t) * E + lane + 64 * j] = a;
    v[j] = lane + 64 * j < E ? a : -INFINITY;
  }
  float gl = 0.0f;
  if (n_gate) {
#pragma unroll
    for (int q = 0; q < KS; ++q) gl += pg[q];
    if (lane == 0) gate[t] = gl;
  }
  uint32_t id;
  float sc;
  topk_wave<NPL>(v, E, k, norm, scr[wave], &id, &sc);
  const int ks = k + m;
  if (lane < k) {
    ids[size_t(t) * ks + lane] = id;
    scores[size_t(t) * ks + lane] = sc;
  } else if (lane < ks) {
    ids[size_t(t) * ks + lane] = uint32_t(E + lane - k);
    scores[size_t(t) * ks + lane] = sigmoidf_(gl);
  }
}

}  // namespace lmoe

using namespace lmoe;

extern "C" int lmoe_grouped_tile_rows(void) { return GM; }

// The tuned tile-row rule (measured on MI355X): 64 when gate/up runs on f16 weights (a type beyond Q4_0 / Q4_K, or
// gate and up of two types: the f16-weight GEMM then fits two workgroups a CU; 2,048 x 8 rows 405 -> 377 us); 64
// for a Q4_K gate/up (the direct-copy kernel k_grouped_q4_k_dma: cfg5 gate/up 545 -> 387 us, and as fast as 128
// rows at 1,000 rows an expert); 128 for a Q4_0 gate/up with an f16 down; 32 when every projection is Q4_0 and an
// expert averages fewer than 16 rows (batched decode: each tile streams its expert's weights, and 32-row tiles keep
// five K steps in flight and allow split-K; cfg4 116.6 -> 108.8 us); else 128.
// LMOE_TILE_ROWS and LMOE_KSPLIT override the two rules below (knobs of the kind of the reference's MOE_GGUF_RUN_TILE,
// gguf_experts.py:590-596, for measuring other tilings). They are read on every call and ignored when the value is
// not one the GEMMs take for these types: tile rows 32 (Q4 projections only), 64 or 128; split-K 1 to 8 slices that
// divide the K steps, on 32-row tiles of at most 65,535 rows.
static int env_knob(const char *name) {
  const char *v = getenv(name);
  return v && *v ? atoi(v) : 0;
}

extern "C" int lmoe_grouped_pick_tile_rows(int R, int E, int type_g, int type_u, int type_d) {
  auto q4 = [](int t) { return t == LMOE_Q4_0 || t == LMOE_Q4_K; };
  const int want = env_knob("LMOE_TILE_ROWS");
  const bool f16w = !(q4(type_g) && type_u == type_g) || !q4(type_d);  // a GEMM on dequantized f16 weights
  if (want == GM || want == 64 || (want == 32 && !f16w)) return want;
  if (!(q4(type_g) && type_u == type_g)) return 64;
  if (type_g == LMOE_Q4_K) return 64;
  if (!q4(type_d)) return GM;
  const bool all_q4_0 = type_g == LMOE_Q4_0 && type_d == LMOE_Q4_0;
  return all_q4_0 && E > 0 && (long long)R < 16LL * E ? 32 : GM;
}

// Split-K slices for one grouped GEMM over K: with 32-row tiles and fewer than 16 rows an expert, few tiles have
// work and each would walk every K step alone, so a tile is split over 4, 3 or 2 workgroups of at least 8 K steps
// each (4 steps of the two-unit GGUF-layout kernel); otherwise 1. Shorter slices lose to the finish kernel they need
// (cfg4's down, 12 K steps: one slice 33.3 us against three slices 30.2 + 4.1 for the finish).
extern "C" int lmoe_grouped_pick_ksplit(int R, int E, int bm, int K) {
  const int steps = K / GK;
  const int want = env_knob("LMOE_KSPLIT");
  if (want == 1 || (want > 1 && want <= 8 && bm == 32 && steps % want == 0 && R <= 65535)) return want;
  if (bm != 32 || E <= 0 || (long long)R >= 16LL * E) return 1;
  for (int s = 4; s >= 2; --s)
    if (steps % (2 * s) == 0 && steps / s >= 8) return s;
  return 1;
}

// Bytes of the split-K workspace (ws) that lmoe_grouped_gate_up_bm and lmoe_grouped_down_bm need over a grouping
// of R rows, E experts and tile rows bm with the picked ksplit of each: ks * R * 2I floats for gate/up, ks * R * H
// for down, the larger of the two (0 when neither splits).
extern "C" size_t lmoe_grouped_workspace_bytes(int R, int E, int bm, int H, int I) {
  if (R <= 0 || H <= 0 || I <= 0) return 0;
  const int ku = lmoe_grouped_pick_ksplit(R, E, bm, H), kd = lmoe_grouped_pick_ksplit(R, E, bm, I);
  const size_t gu = ku > 1 ? size_t(ku) * size_t(R) * 2 * size_t(I) : 0;
  const size_t dn = kd > 1 ? size_t(kd) * size_t(R) * size_t(H) : 0;
  return (gu > dn ? gu : dn) * sizeof(float);
}

static int to_f16(const char *fn, const void *x, int xdtype, long long n, void *out, void *stream, int kperm) {
  LMOE_REQUIRE(dtype_ok(xdtype), LMOE_EINVAL, "%s: bad dtype", fn);
  LMOE_REQUIRE(n >= 0, LMOE_ESHAPE, "%s: negative length", fn);
  LMOE_REQUIRE(!kperm || n % 32 == 0, LMOE_ESHAPE, "%s: length %lld is not a multiple of 32", fn, n);
  if (n == 0) return 0;
  LMOE_REQUIRE(x && out, LMOE_EINVAL, "%s: null pointer", fn);
  const long long blocks = (n + 2047) / 2048;
  LMOE_REQUIRE(blocks < (1ll << 31), LMOE_ESHAPE, "%s: %lld elements", fn, n);
  const int vec = n % 8 == 0 && aligned16(x) && aligned16(out);
  LMOE_REQUIRE(vec || !kperm, LMOE_EALIGN, "%s: x and out must be 16-byte aligned", fn);
  launch(k_to_f16, dim3(unsigned(blocks)), dim3(256), 0, (hipStream_t)stream, x, xdtype, n,
         static_cast<_Float16 *>(out), vec, kperm);
  LMOE_LAUNCHED(fn);
  return 0;
}

extern "C" int lmoe_to_f16(const void *x, int xdtype, long long n, void *out, void *stream) {
  return to_f16("lmoe_to_f16", x, xdtype, n, out, stream, 0);
}

extern "C" int lmoe_to_gemm_f16(const void *x, int xdtype, long long n, void *out, void *stream) {
  return to_f16("lmoe_to_gemm_f16", x, xdtype, n, out, stream, 1);
}

// ksplit > 1: the split-K form (32-row Q4_0 tiles): ksplit workgroups a tile, fp32 slices in ws, then
// k_splitk_finish. Checks shared by both GEMMs.
static int check_split(const char *fn, int bm, int type, int ksplit, const float *ws, int K, int R) {
  LMOE_REQUIRE(ksplit >= 1 && ksplit <= 8, LMOE_ESHAPE, "%s: ksplit %d (1..8)", fn, ksplit);
  if (ksplit == 1) return 0;
  LMOE_REQUIRE(bm == 32 && type == LMOE_Q4_0, LMOE_ESHAPE, "%s: split-K takes 32-row Q4_0 tiles", fn);
  LMOE_REQUIRE((K / GK) % ksplit == 0, LMOE_ESHAPE, "%s: %d K steps do not split in %d", fn, K / GK, ksplit);
  LMOE_REQUIRE(R <= 65535, LMOE_ESHAPE, "%s: %d rows is above the 65535 split-K takes", fn, R);
  LMOE_REQUIRE(ws && aligned16(ws), LMOE_EWORKSPACE, "%s: split-K needs a 16-byte aligned workspace", fn);
  return 0;
}

// The grouped GEMMs' launches. sl: the weights are stream-layout copies (k_stream_repack), which the Q4_0 kernels
// take at every tile height and the Q4_K kernel at 64 rows.
// LDS stages of the 32-row Q4_0 tiles (batched decode: each tile streams one expert's weights): 3 (40 KB, four
// workgroups a CU, two steps in flight) by default; LMOE_Q0_STAGES=4 or 5 trades workgroups for steps in flight
// (53 KB: three a CU; 66 KB: two, four steps ahead). At 3, cfg4's ~620 gate/up tiles run in one wave of workgroups
// instead of a full wave and a ragged second one: 120.4 -> 101.8 us a step on stream copies, 152.2 -> 147.7 on the
// GGUF layout with split-K, the same bits.
static int q0_stages32() {
  const int v = env_knob("LMOE_Q0_STAGES");
  return v == 4 || v == 5 ? v : 3;
}

// The two-unit-step kernel (k_grouped_q4_0_w2) takes the 32-row tiles on the GGUF layout wherever the K steps of
// each slice pair up: its stage count, 2 by default (cfg4 129.8 -> 112.6 us a step, the same bits; 3 stages:
// 116.4), or 0 for the one-unit kernel. LMOE_Q0_W2=1 keeps the one-unit kernel, 3 takes three stages.
// The 64-row Q4_K GEMMs on the GGUF layout stage their weights two steps at a time (k_grouped_q4_k_w2: cfg5 prefill
// 817 -> 761 us, gate/up 421 -> 390, down 252 -> 227, the same bits); LMOE_QK_W2=1 keeps one step at a time.
static bool qk_pairs() { return env_knob("LMOE_QK_W2") != 1; }

// The tall-tile Q4_0 GEMMs on the GGUF layout stage their weights two units at a time (k_grouped_q4_0_p2) where
// K % 128 == 0: cfg3 chunk 750-756 -> 717-721 us (gate/up 414-420 -> 394-405, down 250-261 -> 235-242), the same
// bits. LMOE_Q0_P2=1 keeps the one-unit kernel.
static bool q0_tall_pairs(bool sl, int bm, int K, int ksplit) {
  return !sl && (bm == GM || bm == 64) && ksplit == 1 && (K / GK) % 2 == 0 && env_knob("LMOE_Q0_P2") != 1;
}

static int q0_two_unit(bool sl, int bm, int nst, int K, int ksplit) {
  const int v = env_knob("LMOE_Q0_W2");
  if (sl || bm != 32 || nst != 3 || (K / GK) % (2 * ksplit) != 0 || v == 1) return 0;
  return v == 3 ? 3 : 2;
}

static int grouped_gate_up(const char *fn, bool sl, const void *x, int xdtype, int T, int topk, const uint32_t *order,
                           const uint32_t *offsets, const uint32_t *tiles, const uint32_t *n_tiles, int max_tiles,
                           int bm, int ksplit, float *ws, const uint8_t *wg, const uint8_t *wu, int type_g,
                           int type_u, int n_experts, int H, int I, void *h, void *stream) {
  LMOE_REQUIRE(bm == GM || bm == 64 || bm == 32, LMOE_ESHAPE, "%s: tile rows %d (128, 64 or 32)", fn, bm);
  if (int rc = check_split(fn, bm, type_g, ksplit, ws, H, T * topk)) return rc;
  LMOE_REQUIRE(qtype_ok(type_g) && qtype_ok(type_u), LMOE_ETYPE,
               "%s: ggml types %d/%d are not supported (Q4_0 = 2, Q4_K = 12)", fn, type_g, type_u);
  LMOE_REQUIRE(type_g == type_u, LMOE_ETYPE, "%s: gate and up must share one type on this path (%d vs %d)", fn,
               type_g, type_u);
  LMOE_REQUIRE(!sl || type_g == LMOE_Q4_0 || bm == 64, LMOE_ESHAPE,
               "%s: stream-layout Q4_K weights take 64-row tiles (not %d)", fn, bm);
  LMOE_REQUIRE(xdtype == LMOE_F16, LMOE_EINVAL,
               "%s: x must be float16 in the GEMM K order here (convert once with lmoe_to_gemm_f16)", fn);
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
  const long long grid = (long long)n_ntile * max_tiles * ksplit;
  LMOE_REQUIRE(grid < (1ll << 31), LMOE_ESHAPE, "%s: %lld workgroups", fn, grid);
  hipStream_t st = (hipStream_t)stream;
  const _Float16 *a = static_cast<const _Float16 *>(x);
  if (type_g == LMOE_Q4_0) {
    LMOE_REQUIRE((long long)T * H * 2 <= 0xFFFFFFFFll && (long long)I * (H / 64) * 36 <= 0xFFFFFFFFll, LMOE_ESHAPE,
                 "%s: x or one expert's weights exceed 4 GiB", fn);
    const int R = T * topk;
    const int nst = q0_stages32();
    auto kern = sl ? (bm == 32   ? (nst == 3   ? k_grouped_q4_0<MODE_GATE_UP, 32, 3, true>
                                   : nst == 4 ? k_grouped_q4_0<MODE_GATE_UP, 32, 4, true>
                                              : k_grouped_q4_0<MODE_GATE_UP, 32, 5, true>)
                      : bm == 64 ? k_grouped_q4_0<MODE_GATE_UP, 64, 4, true>
                                 : k_grouped_q4_0<MODE_GATE_UP, GM, 3, true>)
                   : (bm == 32   ? (nst == 3   ? k_grouped_q4_0<MODE_GATE_UP, 32, 3>
                                   : nst == 4 ? k_grouped_q4_0<MODE_GATE_UP, 32, 4>
                                              : k_grouped_q4_0<MODE_GATE_UP, 32, 5>)
                      : bm == 64 ? k_grouped_q4_0<MODE_GATE_UP, 64, 4>
                                 : k_grouped_q4_0<MODE_GATE_UP>);
    if (const int w2 = q0_two_unit(sl, bm, nst, H, ksplit))
      kern = w2 == 2 ? k_grouped_q4_0_w2<MODE_GATE_UP, 32, 2> : k_grouped_q4_0_w2<MODE_GATE_UP, 32, 3>;
    if (q0_tall_pairs(sl, bm, H, ksplit))
      kern = bm == 64 ? k_grouped_q4_0_p2<MODE_GATE_UP, 64> : k_grouped_q4_0_p2<MODE_GATE_UP, GM>;
    launch(kern, dim3(unsigned(grid)), dim3(kThreads), 0, st, a, topk, order, offsets, tiles, n_tiles, n_ntile, wg,
           wu, H, I, h, I, int(LMOE_F16), ksplit, ws, R, 2 * I);
    if (ksplit > 1) {
      LMOE_LAUNCHED(fn);
      launch(k_splitk_finish<MODE_GATE_UP>, dim3(unsigned((I / 4 + 255) / 256), unsigned(R)), dim3(256), 0, st,
             static_cast<const float *>(ws), ksplit, R, 2 * I, offsets, n_experts, h, I, int(LMOE_F16));
    }
  } else {
    launch(sl           ? k_grouped_q4_k_dma<MODE_GATE_UP, 64, 4, true>
           : bm == 32   ? k_grouped_q4_k<MODE_GATE_UP, 32, 3>
           : bm == 64   ? (qk_pairs() ? k_grouped_q4_k_w2<MODE_GATE_UP> : k_grouped_q4_k_dma<MODE_GATE_UP>)
                        : k_grouped_q4_k<MODE_GATE_UP>,
           dim3(unsigned(grid)), dim3(kThreads), 0, st, a, topk, order, offsets, tiles, n_tiles, n_ntile, wg, wu, H,
           I, h, I, int(LMOE_F16));
  }
  LMOE_LAUNCHED(fn);
  return 0;
}

static int grouped_down(const char *fn, bool sl, const void *h, int R, const uint32_t *offsets,
                        const uint32_t *tiles, const uint32_t *n_tiles, int max_tiles, int bm, int ksplit, float *ws,
                        const uint8_t *wd, int type_d, int n_experts, int I, int H, void *y, int ydtype,
                        void *stream) {
  LMOE_REQUIRE(bm == GM || bm == 64 || bm == 32, LMOE_ESHAPE, "%s: tile rows %d (128, 64 or 32)", fn, bm);
  LMOE_REQUIRE(R >= 0, LMOE_ESHAPE, "%s: bad row count", fn);
  if (int rc = check_split(fn, bm, type_d, ksplit, ws, I, R)) return rc;
  LMOE_REQUIRE(qtype_ok(type_d), LMOE_ETYPE, "%s: ggml type %d is not supported (Q4_0 = 2, Q4_K = 12)", fn, type_d);
  LMOE_REQUIRE(!sl || type_d == LMOE_Q4_0 || bm == 64, LMOE_ESHAPE,
               "%s: stream-layout Q4_K weights take 64-row tiles (not %d)", fn, bm);
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
  const long long grid = (long long)n_ntile * max_tiles * ksplit;
  LMOE_REQUIRE(grid < (1ll << 31), LMOE_ESHAPE, "%s: %lld workgroups", fn, grid);
  hipStream_t st = (hipStream_t)stream;
  const _Float16 *a = static_cast<const _Float16 *>(h);
  if (type_d == LMOE_Q4_0) {
    // R is not passed: offsets[E] <= max_tiles * bm rows of h can be read
    LMOE_REQUIRE((long long)max_tiles * bm * I * 2 <= 0xFFFFFFFFll && (long long)H * (I / 64) * 36 <= 0xFFFFFFFFll,
                 LMOE_ESHAPE, "%s: h or one expert's weights exceed 4 GiB", fn);
    const int nst = q0_stages32();
    auto kern = sl ? (bm == 32   ? (nst == 3   ? k_grouped_q4_0<MODE_DOWN, 32, 3, true>
                                   : nst == 4 ? k_grouped_q4_0<MODE_DOWN, 32, 4, true>
                                              : k_grouped_q4_0<MODE_DOWN, 32, 5, true>)
                      : bm == 64 ? k_grouped_q4_0<MODE_DOWN, 64, 4, true>
                                 : k_grouped_q4_0<MODE_DOWN, GM, 3, true>)
                   : (bm == 32   ? (nst == 3   ? k_grouped_q4_0<MODE_DOWN, 32, 3>
                                   : nst == 4 ? k_grouped_q4_0<MODE_DOWN, 32, 4>
                                              : k_grouped_q4_0<MODE_DOWN, 32, 5>)
                      : bm == 64 ? k_grouped_q4_0<MODE_DOWN, 64, 4>
                                 : k_grouped_q4_0<MODE_DOWN>);
    if (const int w2 = q0_two_unit(sl, bm, nst, I, ksplit))
      kern = w2 == 2 ? k_grouped_q4_0_w2<MODE_DOWN, 32, 2> : k_grouped_q4_0_w2<MODE_DOWN, 32, 3>;
    if (q0_tall_pairs(sl, bm, I, ksplit))
      kern = bm == 64 ? k_grouped_q4_0_p2<MODE_DOWN, 64> : k_grouped_q4_0_p2<MODE_DOWN, GM>;
    launch(kern, dim3(unsigned(grid)), dim3(kThreads), 0, st, a, 1, static_cast<const uint32_t *>(nullptr), offsets,
           tiles, n_tiles, n_ntile, wd, static_cast<const uint8_t *>(nullptr), I, H, y, H, ydtype, ksplit, ws, R,
           H);
    if (ksplit > 1) {
      LMOE_LAUNCHED(fn);
      launch(k_splitk_finish<MODE_DOWN>, dim3(unsigned((H / 4 + 255) / 256), unsigned(R)), dim3(256), 0, st,
             static_cast<const float *>(ws), ksplit, R, H, offsets, n_experts, y, H, ydtype);
    }
  } else {
    launch(sl           ? k_grouped_q4_k_dma<MODE_DOWN, 64, 4, true>
           : bm == 32   ? k_grouped_q4_k<MODE_DOWN, 32, 3>
           : bm == 64   ? (qk_pairs() ? k_grouped_q4_k_w2<MODE_DOWN> : k_grouped_q4_k_dma<MODE_DOWN>)
                        : k_grouped_q4_k<MODE_DOWN>,
           dim3(unsigned(grid)), dim3(kThreads), 0, st, a, 1, static_cast<const uint32_t *>(nullptr), offsets, tiles,
           n_tiles, n_ntile, wd, static_cast<const uint8_t *>(nullptr), I, H, y, H, ydtype);
  }
  LMOE_LAUNCHED(fn);
  return 0;
}

extern "C" int lmoe_grouped_gate_up_bm(const void *x, int xdtype, int T, int topk, const uint32_t *order,
                                       const uint32_t *offsets, const uint32_t *tiles, const uint32_t *n_tiles,
                                       int max_tiles, int bm, int ksplit, float *ws, const uint8_t *wg,
                                       const uint8_t *wu, int type_g, int type_u, int n_experts, int H, int I,
                                       void *h, void *stream) {
  return grouped_gate_up("lmoe_grouped_gate_up_bm", false, x, xdtype, T, topk, order, offsets, tiles, n_tiles,
                         max_tiles, bm, ksplit, ws, wg, wu, type_g, type_u, n_experts, H, I, h, stream);
}

extern "C" int lmoe_grouped_gate_up_sl(const void *x, int xdtype, int T, int topk, const uint32_t *order,
                                       const uint32_t *offsets, const uint32_t *tiles, const uint32_t *n_tiles,
                                       int max_tiles, int bm, int ksplit, float *ws, const uint8_t *wg,
                                       const uint8_t *wu, int type_g, int type_u, int n_experts, int H, int I,
                                       void *h, void *stream) {
  return grouped_gate_up("lmoe_grouped_gate_up_sl", true, x, xdtype, T, topk, order, offsets, tiles, n_tiles,
                         max_tiles, bm, ksplit, ws, wg, wu, type_g, type_u, n_experts, H, I, h, stream);
}

extern "C" int lmoe_grouped_down_bm(const void *h, int R, const uint32_t *offsets, const uint32_t *tiles,
                                    const uint32_t *n_tiles, int max_tiles, int bm, int ksplit, float *ws,
                                    const uint8_t *wd, int type_d, int n_experts, int I, int H, void *y, int ydtype,
                                    void *stream) {
  return grouped_down("lmoe_grouped_down_bm", false, h, R, offsets, tiles, n_tiles, max_tiles, bm, ksplit, ws, wd,
                      type_d, n_experts, I, H, y, ydtype, stream);
}

extern "C" int lmoe_grouped_down_sl(const void *h, int R, const uint32_t *offsets, const uint32_t *tiles,
                                    const uint32_t *n_tiles, int max_tiles, int bm, int ksplit, float *ws,
                                    const uint8_t *wd, int type_d, int n_experts, int I, int H, void *y, int ydtype,
                                    void *stream) {
  return grouped_down("lmoe_grouped_down_sl", true, h, R, offsets, tiles, n_tiles, max_tiles, bm, ksplit, ws, wd,
                      type_d, n_experts, I, H, y, ydtype, stream);
}

// Bytes of the stream-layout copy of an expert matrix (the GGUF matrix's own size), or 0 when the shape has no
// stream layout: Q4_0 / Q4_K, rows % 128 == 0, row length a multiple of 64 (Q4_0) or 256 (Q4_K).
extern "C" size_t lmoe_stream_bytes(int type, int n_experts, int rows, int cols) {
  if (!qtype_ok(type) || n_experts <= 0 || rows <= 0 || rows % 128 || cols <= 0 || cols % 64 ||
      cols % block_weights(type))
    return 0;
  return size_t(n_experts) * size_t(rows) * size_t(cols / block_weights(type)) * size_t(type == LMOE_Q4_K ? 144 : 18);
}

extern "C" int lmoe_stream_repack(const uint8_t *src, int type, int n_experts, int rows, int cols, uint8_t *dst,
                                  void *stream) {
  const char *fn = "lmoe_stream_repack";
  LMOE_REQUIRE(qtype_ok(type), LMOE_ETYPE, "%s: ggml type %d has no stream layout (Q4_0 = 2, Q4_K = 12)", fn, type);
  const size_t n = lmoe_stream_bytes(type, n_experts, rows, cols);
  LMOE_REQUIRE(n > 0, LMOE_ESHAPE, "%s: %d experts of %d x %d have no stream layout (rows %% 128, row length %% %d)",
               fn, n_experts, rows, cols, type == LMOE_Q4_K ? 256 : 64);
  LMOE_REQUIRE(src && dst && aligned4(src) && aligned4(dst), LMOE_EALIGN, "%s: 4-byte aligned buffers", fn);
  const long long n_dw = (long long)(n / 4);
  const int row_dw = int(size_t(cols / block_weights(type)) * (type == LMOE_Q4_K ? 144 : 18) / 4);
  const int nkb = type == LMOE_Q4_K ? cols / 256 : cols / 64;
  const long long blocks = (n_dw + 255) / 256;
  LMOE_REQUIRE(blocks < (1ll << 31), LMOE_ESHAPE, "%s: %zu bytes", fn, n);
  auto kern = type == LMOE_Q4_K ? k_stream_repack<LMOE_Q4_K> : k_stream_repack<LMOE_Q4_0>;
  launch(kern, dim3(unsigned(blocks)), dim3(256), 0, (hipStream_t)stream, reinterpret_cast<const uint32_t *>(src),
         rows, row_dw, nkb, n_dw, reinterpret_cast<uint32_t *>(dst));
  LMOE_LAUNCHED(fn);
  return 0;
}

extern "C" int lmoe_grouped_gate_up(const void *x, int xdtype, int T, int topk, const uint32_t *order,
                                    const uint32_t *offsets, const uint32_t *tiles, const uint32_t *n_tiles,
                                    int max_tiles, const uint8_t *wg, const uint8_t *wu, int type_g, int type_u,
                                    int n_experts, int H, int I, void *h, void *stream) {
  return lmoe_grouped_gate_up_bm(x, xdtype, T, topk, order, offsets, tiles, n_tiles, max_tiles, GM, 1, nullptr, wg,
                                 wu, type_g, type_u, n_experts, H, I, h, stream);
}

extern "C" int lmoe_grouped_down(const void *h, const uint32_t *offsets, const uint32_t *tiles,
                                 const uint32_t *n_tiles, int max_tiles, const uint8_t *wd, int type_d, int n_experts,
                                 int I, int H, void *y, int ydtype, void *stream) {
  return lmoe_grouped_down_bm(h, 0, offsets, tiles, n_tiles, max_tiles, GM, 1, nullptr, wd, type_d, n_experts, I, H,
                              y, ydtype, stream);
}

extern "C" int lmoe_grouped_gate_up_f16w(const void *x, int xdtype, int T, int topk, const uint32_t *order,
                                         const uint32_t *offsets, const uint32_t *tiles, const uint32_t *n_tiles,
                                         int max_tiles, int bm, const void *wg16, const void *wu16, int n_experts,
                                         int H, int I, void *h, void *stream) {
  const char *fn = "lmoe_grouped_gate_up_f16w";
  LMOE_REQUIRE(bm == GM || bm == 64, LMOE_ESHAPE, "%s: tile rows %d (128 or 64)", fn, bm);
  LMOE_REQUIRE(xdtype == LMOE_F16, LMOE_EINVAL,
               "%s: x must be float16 in the GEMM K order here (convert once with lmoe_to_gemm_f16)", fn);
  LMOE_REQUIRE(T >= 0 && topk > 0 && n_experts > 0 && max_tiles >= 0, LMOE_ESHAPE, "%s: bad shape", fn);
  LMOE_REQUIRE(H > 0 && H % GK == 0, LMOE_ESHAPE, "%s: hidden size %d is not a multiple of %d", fn, H, GK);
  LMOE_REQUIRE(I > 0 && I % (GN / 2) == 0, LMOE_ESHAPE, "%s: intermediate size %d is not a multiple of %d", fn, I,
               GN / 2);
  if (T == 0 || max_tiles == 0) return 0;
  LMOE_REQUIRE(x && order && offsets && tiles && n_tiles && wg16 && wu16 && h, LMOE_EINVAL, "%s: null pointer", fn);
  LMOE_REQUIRE(aligned16(x) && aligned16(h) && aligned16(wg16) && aligned16(wu16), LMOE_EALIGN,
               "%s: x, h and the weights must be 16-byte aligned", fn);
  LMOE_REQUIRE((long long)T * H * 2 <= 0xFFFFFFFFll && (long long)I * H * 2 <= 0xFFFFFFFFll, LMOE_ESHAPE,
               "%s: x or one expert's weights exceed 4 GiB", fn);
  const int n_ntile = I / (GN / 2);
  const long long grid = (long long)n_ntile * max_tiles;
  LMOE_REQUIRE(grid < (1ll << 31), LMOE_ESHAPE, "%s: %lld workgroups", fn, grid);
  launch(bm == 64 ? k_grouped_f16w<MODE_GATE_UP, 64> : k_grouped_f16w<MODE_GATE_UP>, dim3(unsigned(grid)),
         dim3(kThreads), 0, (hipStream_t)stream,
         static_cast<const _Float16 *>(x), topk, order, offsets, tiles, n_tiles, n_ntile,
         static_cast<const _Float16 *>(wg16), static_cast<const _Float16 *>(wu16), H, I, h, I, int(LMOE_F16));
  LMOE_LAUNCHED(fn);
  return 0;
}

extern "C" int lmoe_grouped_down_f16w(const void *h, const uint32_t *offsets, const uint32_t *tiles,
                                      const uint32_t *n_tiles, int max_tiles, int bm, const void *wd16, int n_experts,
                                      int I, int H, void *y, int ydtype, void *stream) {
  const char *fn = "lmoe_grouped_down_f16w";
  LMOE_REQUIRE(bm == GM || bm == 64, LMOE_ESHAPE, "%s: tile rows %d (128 or 64)", fn, bm);
  LMOE_REQUIRE(n_experts > 0 && max_tiles >= 0, LMOE_ESHAPE, "%s: bad shape", fn);
  LMOE_REQUIRE(I > 0 && I % GK == 0, LMOE_ESHAPE, "%s: intermediate size %d is not a multiple of %d", fn, I, GK);
  LMOE_REQUIRE(H > 0 && H % GN == 0, LMOE_ESHAPE, "%s: hidden size %d is not a multiple of %d", fn, H, GN);
  LMOE_REQUIRE(ydtype == LMOE_F16 || ydtype == LMOE_F32, LMOE_EINVAL, "%s: y must be float16 or float32", fn);
  if (max_tiles == 0) return 0;
  LMOE_REQUIRE(h && offsets && tiles && n_tiles && wd16 && y, LMOE_EINVAL, "%s: null pointer", fn);
  LMOE_REQUIRE(aligned16(h) && aligned16(y) && aligned16(wd16), LMOE_EALIGN,
               "%s: h, y and the weights must be 16-byte aligned", fn);
  // R is not passed: offsets[E] <= max_tiles * bm rows of h can be read
  LMOE_REQUIRE((long long)max_tiles * bm * I * 2 <= 0xFFFFFFFFll && (long long)H * I * 2 <= 0xFFFFFFFFll,
               LMOE_ESHAPE, "%s: h or one expert's weights exceed 4 GiB", fn);
  const int n_ntile = H / GN;
  const long long grid = (long long)n_ntile * max_tiles;
  LMOE_REQUIRE(grid < (1ll << 31), LMOE_ESHAPE, "%s: %lld workgroups", fn, grid);
  launch(bm == 64 ? k_grouped_f16w<MODE_DOWN, 64> : k_grouped_f16w<MODE_DOWN>, dim3(unsigned(grid)), dim3(kThreads),
         0, (hipStream_t)stream,
         static_cast<const _Float16 *>(h), 1, static_cast<const uint32_t *>(nullptr), offsets, tiles, n_tiles, n_ntile,
         static_cast<const _Float16 *>(wd16), static_cast<const _Float16 *>(nullptr), I, H, y, H, ydtype);
  LMOE_LAUNCHED(fn);
  return 0;
}

// The prefill router's split: K slices so that at least ~512 workgroups run, each slice at least 4 K steps, the
// slice count a power of two dividing the K steps
extern "C" int lmoe_router_gemm_ksplit(int T, int H, int En) {
  if (T <= 0 || H <= 0 || En <= 0) return 1;
  const long long tiles = (long long)((T + kRgM - 1) / kRgM) * ((En + kRgN - 1) / kRgN);
  const int steps = H / GK;
  int s = 1;
  while (tiles * s < 512 && s < 8 && steps % (2 * s) == 0 && steps / (2 * s) >= 4) s *= 2;
  return s;
}

extern "C" size_t lmoe_router_gemm_workspace_bytes(int T, int H, int En) {
  const int s = lmoe_router_gemm_ksplit(T, H, En);
  if (s <= 1) return 0;
  return size_t(s) * size_t(T) * size_t((En + kRgN - 1) / kRgN * kRgN) * sizeof(float);
}

// The router GEMM's launch; with finish false and a K split, the slices stay in ws for the caller (*ks_out, *ldp_out).
// split_rows (> 0): the row count the K split is chosen for, in place of E + n_gate.
static int router_gemm(const char *fn, const void *xh, int T, int H, const void *wk, int E, int n_gate, float *ws,
                       float *logits, float *gate, bool finish, int *ks_out, int *ldp_out, hipStream_t st,
                       int split_rows = 0) {
  LMOE_REQUIRE(T >= 0 && E > 0 && (n_gate == 0 || n_gate == 1), LMOE_ESHAPE, "%s: bad shape", fn);
  LMOE_REQUIRE(H > 0 && H % GK == 0, LMOE_ESHAPE, "%s: hidden size %d is not a multiple of %d", fn, H, GK);
  if (T == 0) return 0;
  LMOE_REQUIRE(xh && wk && logits && (n_gate == 0 || gate), LMOE_EINVAL, "%s: null pointer", fn);
  LMOE_REQUIRE(aligned16(xh) && aligned16(wk), LMOE_EALIGN, "%s: x and the weight must be 16-byte aligned", fn);
  const int En = E + n_gate;
  LMOE_REQUIRE((long long)T * H * 2 <= 0xFFFFFFFFll && (long long)En * H * 2 <= 0xFFFFFFFFll, LMOE_ESHAPE,
               "%s: x or the weight exceeds 4 GiB", fn);
  const int ks = lmoe_router_gemm_ksplit(T, H, split_rows > 0 ? split_rows : En);
  const int n_ntile = (En + kRgN - 1) / kRgN, ldp = n_ntile * kRgN;
  LMOE_REQUIRE(ks == 1 || (ws && aligned16(ws)), LMOE_EWORKSPACE,
               "%s: needs a 16-byte aligned workspace of lmoe_router_gemm_workspace_bytes", fn);
  const long long grid = (long long)((T + kRgM - 1) / kRgM) * n_ntile * ks;
  LMOE_REQUIRE(grid < (1ll << 31), LMOE_ESHAPE, "%s: %lld workgroups", fn, grid);
  launch(k_router_gemm, dim3(unsigned(grid)), dim3(kThreads), 0, st, static_cast<const _Float16 *>(xh), T,
         static_cast<const _Float16 *>(wk), En, H, n_ntile, ks, ws, ldp, logits, E, gate);
  if (ks > 1 && finish) {
    LMOE_LAUNCHED(fn);
    launch(k_router_finish, dim3(unsigned((En + 255) / 256), unsigned(T)), dim3(256), 0, st,
           static_cast<const float *>(ws), ks, T, ldp, En, E, logits, gate);
  }
  LMOE_LAUNCHED(fn);
  *ks_out = ks;
  *ldp_out = ldp;
  return 0;
}

extern "C" int lmoe_router_gemm(const void *xh, int T, int H, const void *wk, int E, int n_gate, float *ws,
                                float *logits, float *gate, void *stream) {
  int ks, ldp;
  return router_gemm("lmoe_router_gemm", xh, T, H, wk, E, n_gate, ws, logits, gate, true, &ks, &ldp,
                     (hipStream_t)stream);
}

extern "C" int lmoe_router_refine(const float *part, int ksplit, int ldp, const void *x, int xdtype, int T, int H,
                                  const void *wr, const void *wsg, int wdtype, int E, const float *norms, int k,
                                  int norm, int m, uint32_t *ids, float *scores, float *logits, float *gate,
                                  int *n_cand, void *stream);

// The router GEMM, then its picks made exact by lmoe_router_refine (refine.hip) straight from the K slices (or the
// logits, unsplit): ids equal to the top-k of the decode router's fixed-order logits on the same x. The shared
// expert's gate row is left out of the GEMM: the refine recomputes it in the fixed order for every token (at E = 512
// that row alone was a fifth of the GEMM's tiles). The K split is still chosen for E + n_gate rows, so the slices,
// and everything the refine derives from them, are those of the GEMM with the row.
extern "C" int lmoe_router_gemm_refine(const void *xh, int T, int H, const void *wk, int E, int n_gate, float *ws,
                                       const void *x, int xdtype, const void *wr, const void *wsg, int wdtype,
                                       const float *norms, int k, int norm, int m, uint32_t *ids, float *scores,
                                       float *logits, float *gate, int *n_cand, void *stream) {
  const char *fn = "lmoe_router_gemm_refine";
  LMOE_REQUIRE((n_gate == 1) == (wsg != nullptr), LMOE_EINVAL, "%s: the gate row and wsg go together", fn);
  hipStream_t st = (hipStream_t)stream;
  int ks = 1, ldp = 0;
  if (int rc = router_gemm(fn, xh, T, H, wk, E, 0, ws, logits, nullptr, false, &ks, &ldp, st, E + n_gate)) return rc;
  if (T == 0) return 0;
  return lmoe_router_refine(ks > 1 ? ws : logits, ks, ks > 1 ? ldp : E, x, xdtype, T, H, wr, wsg, wdtype, E, norms,
                            k, norm, m, ids, scores, logits, gate, n_cand, stream);
}

extern "C" int lmoe_router_gemm_topk(const void *xh, int T, int H, const void *wk, int E, int n_gate, float *ws,
                                     float *logits, float *gate, int k, int norm, int m, uint32_t *ids,
                                     float *scores, void *stream) {
  const char *fn = "lmoe_router_gemm_topk";
  LMOE_REQUIRE(E > 0 && E <= 1024, LMOE_ESHAPE, "%s: %d experts is outside 1..1024", fn, E);
  LMOE_REQUIRE(k > 0 && k <= E && k <= 32 && m >= 0 && k + m <= 64, LMOE_ESHAPE,
               "%s: top-k %d with %d shared slices is outside what the top-k takes", fn, k, m);
  LMOE_REQUIRE(m == 0 || n_gate == 1, LMOE_EINVAL, "%s: shared slices need the gate row", fn);
  LMOE_REQUIRE(T == 0 || (ids && scores), LMOE_EINVAL, "%s: null pointer", fn);
  hipStream_t st = (hipStream_t)stream;
  int ks = 1, ldp = 0;
  if (int rc = router_gemm(fn, xh, T, H, wk, E, n_gate, ws, logits, gate, false, &ks, &ldp, st)) return rc;
  if (T == 0) return 0;
  if (ks == 1)  // the GEMM wrote the logits (and the gate logit) itself: the plain top-k on them
    return m > 0 ? lmoe_router_topk_shared(logits, T, E, k, norm, gate, m, ids, scores, stream)
                 : lmoe_router_topk(logits, LMOE_F32, T, E, k, norm, ids, scores, stream);
  const dim3 grid((T + 3) / 4), block(256);
  const float *pw = static_cast<const float *>(ws);
  auto by_ks = [&](auto npl, auto ksc) {
    constexpr int N = decltype(npl)::value, K = decltype(ksc)::value;
    launch(k_topk_from_parts<N, K>, grid, block, 0, st, pw, T, ldp, E, n_gate, k, norm, m, logits, gate, ids,
           scores);
  };
  auto go = [&](auto npl) {
    if (ks == 2) by_ks(npl, IC<2>{});
    else if (ks == 4) by_ks(npl, IC<4>{});
    else by_ks(npl, IC<8>{});
  };
  LMOE_REQUIRE(ks == 2 || ks == 4 || ks == 8, LMOE_ESHAPE, "%s: K split %d", fn, ks);
  if (E <= 64) go(IC<1>{});
  else if (E <= 128) go(IC<2>{});
  else if (E <= 256) go(IC<4>{});
  else if (E <= 512) go(IC<8>{});
  else go(IC<16>{});
  LMOE_LAUNCHED(fn);
  return 0;
}
