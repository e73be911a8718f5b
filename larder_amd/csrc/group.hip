// Device-side ragged grouping: a stable counting sort of the flattened (token, k) expert ids.
//
// The reference groups on the host: mx.argsort of the flat ids and its inverse (stream_fast.py:5466-5471), then
// np.unique / searchsorted between units (gguf_experts.py:702-713; stream_fast.py:92-122), with an mx.eval sync
// each layer. Here three kernels do it on the device with no host round trip, for R rows in chunks of 256:
//   1. k_group_count: each workgroup histograms its chunk in LDS and writes the counts bucket-major,
//      hist[bucket][chunk];
//   2. k_group_scan: one workgroup a bucket turns its row of hist into the exclusive prefix over chunks (the
//      bucket's rows in earlier chunks) and writes the bucket total;
//   3. k_group_scatter: each workgroup scans the totals into bucket offsets, and every row goes to
//      offset[bucket] + rows of its bucket in earlier chunks + rows of its bucket earlier in its own chunk (its rank
//      inside its wavefront by ballots, plus the bucket's rows in the chunk's earlier wavefronts), so rows keep flat
//      order within an expert. Workgroup 0 also
//      writes counts, offsets and the grouped GEMM's work list.
// Bucket E collects ids >= E, which therefore sort after every expert.
#include <cstdlib>
#include <mutex>

#include "lmoe_common.h"

namespace lmoe {

constexpr int kGroupChunk = 256;
constexpr int kGroupMaxE = 1024;

// exclusive prefix sum of v over the 256 threads of the block; *total gets the sum. tmp: 4 words of LDS.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t *tmp, uint32_t *total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint32_t x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) tmp[wave] = x;
  __syncthreads();
  uint32_t base = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t t = tmp[w];
    base += w < wave ? t : 0u;
    tot += t;
  }
  __syncthreads();
  *total = tot;
  return base + x - v;
}

__global__ void __launch_bounds__(256) k_group_count(const uint32_t *ids, int R, int E, int nchunk,
                                                      uint32_t *hist) {
  __shared__ uint32_t cnt[kGroupMaxE + 1];
  for (int e = threadIdx.x; e <= E; e += 256) cnt[e] = 0;
  __syncthreads();
  const int r = blockIdx.x * kGroupChunk + threadIdx.x;
  if (r < R) {
    const uint32_t v = ids[r];
    atomicAdd(&cnt[v < uint32_t(E) ? v : uint32_t(E)], 1u);
  }
  __syncthreads();
  for (int e = threadIdx.x; e <= E; e += 256) hist[size_t(e) * nchunk + blockIdx.x] = cnt[e];
}

// grid E + 1: bucket blockIdx.x
__global__ void __launch_bounds__(256) k_group_scan(int nchunk, uint32_t *hist, uint32_t *totals) {
  __shared__ uint32_t tmp[4];
  uint32_t *row = hist + size_t(blockIdx.x) * nchunk;
  uint32_t carry = 0;
  for (int c0 = 0; c0 < nchunk; c0 += 256) {
    const int c = c0 + threadIdx.x;
    const uint32_t v = c < nchunk ? row[c] : 0u;
    uint32_t tot;
    const uint32_t ex = block_exclusive_scan(v, tmp, &tot);
    if (c < nchunk) row[c] = carry + ex;
    carry += tot;
  }
  if (threadIdx.x == 0) totals[blockIdx.x] = carry;
}

__global__ void __launch_bounds__(256)
    k_group_scatter(const uint32_t *ids, int R, int E, int bm, const uint32_t *hist, const uint32_t *totals,
                    int nchunk, uint32_t *counts, uint32_t *offsets, uint32_t *order, uint32_t *inv, uint32_t *tiles,
                    uint32_t *n_tiles) {
  __shared__ uint32_t off[kGroupMaxE + 1];
  __shared__ uint8_t wc[4][kGroupMaxE + 4];  // rows of bucket e in wavefront w of the chunk (<= 64)
  __shared__ uint32_t tmp[4];
  const int c = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // bucket offsets: exclusive scan of the totals, 4 consecutive buckets a thread (E + 1 <= 1025 < 1028)
  {
    uint32_t t[4], sum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = 4 * tid + i;
      t[i] = e <= E ? totals[e] : 0u;
      sum += t[i];
    }
    uint32_t tot;
    uint32_t run = block_exclusive_scan(sum, tmp, &tot);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = 4 * tid + i;
      if (e <= E) off[e] = run;
      run += t[i];
    }
  }
  __syncthreads();
  if (E == kGroupMaxE) {  // the 1025th bucket (ids >= 1024) falls outside the 4-a-thread scan
    if (tid == 0) off[kGroupMaxE] = off[kGroupMaxE - 1] + totals[kGroupMaxE - 1];
    __syncthreads();
  }
  if (c == 0) {
    for (int e = tid; e < E; e += 256) counts[e] = totals[e];
    for (int e = tid; e <= E; e += 256) offsets[e] = off[e];
    if (tiles) {  // the work list: each expert's m-tiles in order, experts ascending
      const int per = (E + 255) / 256;  // experts a thread: tid * per ..
      uint32_t nt[4] = {0, 0, 0, 0}, sum = 0;
      for (int i = 0; i < per; ++i) {
        const int e = tid * per + i;
        nt[i] = e < E ? (totals[e] + uint32_t(bm) - 1) / uint32_t(bm) : 0u;
        sum += nt[i];
      }
      uint32_t tot;
      uint32_t run = block_exclusive_scan(sum, tmp, &tot);
      for (int i = 0; i < per; ++i) {
        const int e = tid * per + i;
        for (uint32_t m = 0; m < nt[i]; ++m) tiles[run + m] = (uint32_t(e) << 20) | m;
        run += nt[i];
      }
      if (tid == 0) *n_tiles = tot;
    }
  }
  const int r = c * kGroupChunk + tid;
  const bool act = r < R;
  uint32_t key = uint32_t(E);
  if (act) {
    const uint32_t v = ids[r];
    key = v < uint32_t(E) ? v : uint32_t(E);
  }
  // rows of this bucket earlier in the chunk: the row's rank inside its wavefront (a ballot for each distinct key
  // of the wavefront) plus the bucket's rows in the chunk's earlier wavefronts
  for (int i = tid; i < 4 * (kGroupMaxE + 4) / 4; i += 256) reinterpret_cast<uint32_t *>(wc)[i] = 0;
  __syncthreads();
  const uint64_t below = (uint64_t(1) << lane) - 1;
  uint32_t rank = 0;
  uint64_t rem = __ballot(act);
  while (rem) {
    const uint32_t lk = uint32_t(__builtin_amdgcn_readlane(int(key), __builtin_ctzll(rem)));
    const uint64_t m = __ballot(act && key == lk);
    if (act && key == lk) {
      rank = uint32_t(__popcll(m & below));
      if (rank == 0) wc[wave][lk] = uint8_t(__popcll(m));
    }
    rem &= ~m;
  }
  __syncthreads();
  if (!act) return;
  for (int w = 0; w < wave; ++w) rank += wc[w][key];
  const uint32_t pos = off[key] + hist[size_t(key) * nchunk + c] + rank;
  order[pos] = uint32_t(r);
  inv[r] = pos;
}

// ---- the same sort for R <= 1024 rows in one workgroup -----------------------------------------------------------
//
// One row a thread, 16 wavefronts: the histogram and its exclusive scan in LDS; each row's rank among the earlier
// rows of its bucket is its rank inside its wavefront (a ballot for each distinct key of the wavefront, lowest lane
// first) plus the rows of that bucket in the earlier wavefronts (per-wavefront bucket counts in LDS, 16 x 1025
// bytes). The same positions as the three kernels (a stable sort), in one launch and with no serial loop over rows.
constexpr int kGroupSmallR = 1024;

__global__ void __launch_bounds__(1024)
    k_group_small(const uint32_t *ids, int R, int E, int bm, uint32_t *counts, uint32_t *offsets, uint32_t *order,
                  uint32_t *inv, uint32_t *tiles, uint32_t *n_tiles) {
  __shared__ uint32_t cnt[kGroupMaxE + 1];  // bucket counts, then their exclusive prefix
  __shared__ uint8_t wc[16][kGroupMaxE + 4];  // rows of bucket e in wavefront w (<= 64)
  __shared__ uint32_t wsum[16], wsum2[16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int e = tid; e <= E; e += 1024) cnt[e] = 0;
  for (int i = tid; i < 16 * (kGroupMaxE + 4) / 4; i += 1024) reinterpret_cast<uint32_t *>(wc)[i] = 0;
  __syncthreads();
  const bool act = tid < R;
  uint32_t key = uint32_t(E);
  if (act) {
    const uint32_t v = ids[tid];
    key = v < uint32_t(E) ? v : uint32_t(E);
    atomicAdd(&cnt[key], 1u);
  }
  // rank inside the wavefront and the wavefront's count of each key: one ballot a distinct key
  const uint64_t below = (uint64_t(1) << lane) - 1;
  uint32_t wrank = 0;
  uint64_t rem = __ballot(act);
  while (rem) {
    const uint32_t lk = uint32_t(__builtin_amdgcn_readlane(int(key), __builtin_ctzll(rem)));
    const uint64_t m = __ballot(act && key == lk);
    if (act && key == lk) {
      wrank = uint32_t(__popcll(m & below));
      if (wrank == 0) wc[wave][lk] = uint8_t(__popcll(m));
    }
    rem &= ~m;
  }
  __syncthreads();
  // exclusive scan of the bucket counts: bucket tid (bucket 1024, when E == 1024, added after)
  uint32_t c = tid <= E ? cnt[tid] : 0u, x = c;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) wsum[wave] = x;
  // experts' m-tiles for the work list: the same scan over ceil(count / bm)
  const uint32_t nt = tiles && tid < E ? (c + uint32_t(bm) - 1) / uint32_t(bm) : 0u;
  uint32_t xt = nt;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(xt, o, 64);
    if (lane >= o) xt += y;
  }
  if (lane == 63) wsum2[wave] = xt;
  __syncthreads();
  uint32_t base = 0, tbase = 0, ttot = 0;
  for (int w = 0; w < 16; ++w) {
    base += w < wave ? wsum[w] : 0u;
    tbase += w < wave ? wsum2[w] : 0u;
    ttot += wsum2[w];
  }
  const uint32_t off = base + x - c;  // bucket tid's first position
  if (tid <= E) {
    if (tid < E) counts[tid] = c;
    offsets[tid] = off;
  }
  if (E == kGroupMaxE && tid == 1023) offsets[kGroupMaxE] = off + c;  // bucket 1024 starts after bucket 1023
  if (tiles) {
    uint32_t run = tbase + xt - nt;
    for (uint32_t m = 0; m < nt; ++m) tiles[run + m] = (uint32_t(tid) << 20) | m;
    if (tid == 0) *n_tiles = ttot;
  }
  __syncthreads();  // every thread has read cnt: it becomes the offsets
  if (tid <= E) cnt[tid] = off;
  if (E == kGroupMaxE && tid == 1023) cnt[kGroupMaxE] = off + c;
  __syncthreads();
  if (!act) return;
  uint32_t pos = cnt[key] + wrank;
  for (int w = 0; w < wave; ++w) pos += wc[w][key];
  order[pos] = uint32_t(tid);
  inv[tid] = pos;
}

}  // namespace lmoe

using namespace lmoe;

extern "C" size_t lmoe_group_workspace_bytes(int R, int E) {
  const size_t nchunk = (size_t(R > 0 ? R : 1) + kGroupChunk - 1) / kGroupChunk;
  return (nchunk + 1) * size_t(E + 1) * 4;
}

extern "C" int lmoe_max_tiles(int R, int E, int bm) { return bm > 0 ? (R + bm - 1) / bm + E : 0; }

// R <= 1024 rows go through k_group_small unless LMOE_GROUP_SMALL=0
static bool small_grouping() {
  static const bool on = [] {
    const char *v = getenv("LMOE_GROUP_SMALL");
    return !(v && v[0] == '0');
  }();
  return on;
}

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
  if (R <= kGroupSmallR && small_grouping()) {  // one launch
    launch(k_group_small, dim3(1), dim3(1024), 0, st, ids, R, E, bm, counts, offsets, order, inv, tiles, n_tiles);
    LMOE_LAUNCHED(fn);
    return 0;
  }
  const int nchunk = R > 0 ? (R + kGroupChunk - 1) / kGroupChunk : 1;
  uint32_t *hist = static_cast<uint32_t *>(ws);
  uint32_t *totals = hist + size_t(nchunk) * (E + 1);
  launch(k_group_count, dim3(nchunk), dim3(256), 0, st, ids, R, E, nchunk, hist);
  LMOE_LAUNCHED(fn);
  launch(k_group_scan, dim3(E + 1), dim3(256), 0, st, nchunk, hist, totals);
  LMOE_LAUNCHED(fn);
  launch(k_group_scatter, dim3(nchunk), dim3(256), 0, st, ids, R, E, bm, static_cast<const uint32_t *>(hist),
         static_cast<const uint32_t *>(totals), nchunk, counts, offsets, order, inv, tiles, n_tiles);
  LMOE_LAUNCHED(fn);
  return 0;
}

// ---- the same grouping with no caller workspace ------------------------------------------------------------------
//
// For callers that cannot allocate device memory (code under graph capture, serving loops, harnesses that forbid
// it): the histograms and totals live in a file-scope device array. Each GPU holds its own copy until the process
// ends; its address is taken once per device (hipGetSymbolAddress) and kept, and host code passes only that address
// to kernels. Every call on one GPU shares the array, so calls that overlap on one GPU race. The count and scan
// kernels write every entry they later read, so nothing needs clearing between calls.
namespace lmoe {
constexpr size_t kGroupScratchBytes = size_t(1) << 20;
static __device__ __align__(256) uint8_t scratch[kGroupScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

int scratch_for_current_device(void **out, const char *fn) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, fn);
  LMOE_REQUIRE(dev >= 0 && dev < kMaxDevices, LMOE_EINVAL, "%s: device %d is past %d", fn, dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, fn);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}
}  // namespace
}  // namespace lmoe

extern "C" int lmoe_group_rows_noalloc(const uint32_t *ids, int R, int E, int bm, uint32_t *counts,
                                       uint32_t *offsets, uint32_t *order, uint32_t *inv, uint32_t *tiles,
                                       uint32_t *n_tiles, void *stream) {
  const char *fn = "lmoe_group_rows_noalloc";
  LMOE_REQUIRE(R >= 0 && R <= (1 << 24), LMOE_ESHAPE, "%s: %d rows is outside 0..2^24", fn, R);
  LMOE_REQUIRE(E > 0 && E <= kGroupMaxE, LMOE_ESHAPE, "%s: %d experts is outside 1..%d", fn, E, kGroupMaxE);
  const size_t need = lmoe_group_workspace_bytes(R, E);
  LMOE_REQUIRE(need <= kGroupScratchBytes, LMOE_EWORKSPACE,
               "%s: %d rows over %d experts need %zu bytes of scratch, more than the %zu this entry point holds", fn,
               R, E, need, kGroupScratchBytes);
  void *ws = nullptr;
  if (int rc = scratch_for_current_device(&ws, fn)) return rc;
  return lmoe_group_rows(ids, R, E, bm, counts, offsets, order, inv, tiles, n_tiles, ws, stream);
}
