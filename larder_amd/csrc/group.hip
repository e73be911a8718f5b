// Device-side ragged grouping: a stable counting sort of the flattened (token, k) expert ids.
//
// The reference groups on the host: mx.argsort of the flat ids and its inverse (stream_fast.py:5466-5471), then
// np.unique / searchsorted between units (gguf_experts.py:702-713; stream_fast.py:92-122), with an mx.eval sync
// each layer. Here two kernels do it on the device with no host round trip:
//   1. k_group_hist: each workgroup histograms one chunk of CH rows into LDS and writes its counts;
//   2. k_group_scatter: each workgroup derives its chunk's start in every bucket from the counts of the chunks
//      before it (so the sort is stable across chunks), then one wavefront walks its chunk 64 rows at a time,
//      ranking equal ids inside a group of 64 by ballot, so rows keep flat order within an expert.
// Workgroup 0 also writes counts, offsets and the grouped GEMM's work list.
#include "lmoe_common.h"

namespace lmoe {

constexpr int kGroupChunk = 512;
constexpr int kGroupMaxE = 1024;

__global__ void __launch_bounds__(256) k_group_hist(const uint32_t *ids, int R, int E, uint32_t *hist) {
  __shared__ uint32_t cnt[kGroupMaxE + 1];
  for (int e = threadIdx.x; e <= E; e += 256) cnt[e] = 0;
  __syncthreads();
  const int r0 = blockIdx.x * kGroupChunk, r1 = min(R, r0 + kGroupChunk);
  for (int r = r0 + threadIdx.x; r < r1; r += 256) {
    const uint32_t v = ids[r];
    atomicAdd(&cnt[v < uint32_t(E) ? v : uint32_t(E)], 1u);
  }
  __syncthreads();
  for (int e = threadIdx.x; e <= E; e += 256) hist[size_t(blockIdx.x) * (E + 1) + e] = cnt[e];
}

__global__ void __launch_bounds__(256)
    k_group_scatter(const uint32_t *ids, int R, int E, int bm, const uint32_t *hist, int nchunk, uint32_t *counts,
                    uint32_t *offsets, uint32_t *order, uint32_t *inv, uint32_t *tiles, uint32_t *n_tiles) {
  __shared__ uint32_t base[kGroupMaxE + 1];
  __shared__ uint32_t tot[kGroupMaxE + 1];
  const int c = blockIdx.x;
  // per bucket: rows in all chunks (tot) and rows in chunks before this one (base)
  for (int e = threadIdx.x; e <= E; e += 256) {
    uint32_t before = 0, all = 0;
    for (int j = 0; j < nchunk; ++j) {
      const uint32_t v = hist[size_t(j) * (E + 1) + e];
      all += v;
      before += j < c ? v : 0u;
    }
    tot[e] = all;
    base[e] = before;
  }
  __syncthreads();
  if (threadIdx.x == 0) {  // exclusive scan over buckets (E + 1 of them: the last holds ids >= E)
    uint32_t run = 0;
    for (int e = 0; e <= E; ++e) {
      const uint32_t v = tot[e];
      tot[e] = run;
      run += v;
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e <= E; e += 256) base[e] += tot[e];
  if (c == 0) {
    for (int e = threadIdx.x; e < E; e += 256) counts[e] = tot[e + 1] - tot[e];
    for (int e = threadIdx.x; e <= E; e += 256) offsets[e] = tot[e];
    if (threadIdx.x == 0 && tiles) {
      uint32_t nt = 0;
      for (int e = 0; e < E; ++e) {
        const uint32_t n = tot[e + 1] - tot[e];
        for (uint32_t m = 0; m * uint32_t(bm) < n; ++m) tiles[nt++] = (uint32_t(e) << 20) | m;
      }
      *n_tiles = nt;
    }
  }
  __syncthreads();
  if (threadIdx.x >= 64) return;
  const int lane = threadIdx.x;
  const int r0 = c * kGroupChunk, r1 = min(R, r0 + kGroupChunk);
  for (int g = r0; g < r1; g += 64) {
    const int r = g + lane;
    const bool act = r < r1;
    const uint32_t v = act ? ids[r] : 0u;
    const uint32_t key = v < uint32_t(E) ? v : uint32_t(E);
    uint64_t pending = __ballot(act);
    uint32_t pos = 0;
    while (pending) {
      const int leader = __ffsll((unsigned long long)pending) - 1;
      const uint32_t k0 = __shfl(key, leader, 64);
      const uint64_t same = __ballot(act && key == k0);
      if (act && key == k0) {
        const uint64_t below = same & ((uint64_t(1) << lane) - 1);
        pos = base[k0] + __popcll(below);
      }
      if (lane == leader) base[k0] += __popcll(same);
      pending &= ~same;
      __builtin_amdgcn_wave_barrier();
    }
    if (act) {
      order[pos] = uint32_t(r);
      inv[r] = pos;
    }
  }
}

}  // namespace lmoe

using namespace lmoe;

extern "C" size_t lmoe_group_workspace_bytes(int R, int E) {
  const size_t nchunk = (size_t(R > 0 ? R : 1) + kGroupChunk - 1) / kGroupChunk;
  return nchunk * size_t(E + 1) * 4;
}

extern "C" int lmoe_max_tiles(int R, int E, int bm) { return bm > 0 ? (R + bm - 1) / bm + E : 0; }

extern "C" int lmoe_group_rows(const uint32_t *ids, int R, int E, int bm, uint32_t *counts, uint32_t *offsets,
                               uint32_t *order, uint32_t *inv, uint32_t *tiles, uint32_t *n_tiles, void *ws,
                               void *stream) {
  const char *fn = "lmoe_group_rows";
  LMOE_REQUIRE(R >= 0 && R <= (1 << 24), LMOE_ESHAPE, "%s: %d rows is outside 0..2^24", fn, R);
  LMOE_REQUIRE(E > 0 && E <= kGroupMaxE, LMOE_ESHAPE, "%s: %d experts is outside 1..%d", fn, E, kGroupMaxE);
  LMOE_REQUIRE(!tiles || (bm >= 16 && n_tiles), LMOE_EINVAL, "%s: tiles need bm >= 16 and n_tiles", fn);
  LMOE_REQUIRE(counts && offsets && ws, LMOE_EINVAL, "%s: null pointer", fn);
  LMOE_REQUIRE(R == 0 || (ids && order && inv), LMOE_EINVAL, "%s: null pointer", fn);
  hipStream_t st = (hipStream_t)stream;
  const int nchunk = R > 0 ? (R + kGroupChunk - 1) / kGroupChunk : 1;
  uint32_t *hist = static_cast<uint32_t *>(ws);
  launch(k_group_hist, dim3(nchunk), dim3(256), 0, st, ids, R, E, hist);
  LMOE_LAUNCHED(fn);
  launch(k_group_scatter, dim3(nchunk), dim3(256), 0, st, ids, R, E, bm, hist, nchunk, counts, offsets,
                     order, inv, tiles, n_tiles);
  LMOE_LAUNCHED(fn);
  return 0;
}
