// Batch-1 decode through a stack of MoE layers as ONE persistent cooperative kernel.
//
// The per-layer chain (router GEMV -> top-k -> gate/up + SwiGLU -> down + combine + residual) has three
// all-to-all dependencies a layer: every expert row needs all of x, every top-k needs all router logits, every
// output row needs all of h. As separate kernels each costs a dependent launch (1.6-1.7 us on MI355X inside a HIP
// graph, measured) plus the new grid's ramp and first-load latency. Here one workgroup a CU stays resident for the
// whole stack and the dependencies go through memory:
//   * every exchanged value travels in a 64-bit word (payload | epoch << 32), written with one device-coherent
//     store and read with device-coherent loads; a reader polls its words until all carry this launch's epoch, so
//     no counter, fence or barrier is involved and a hand-off costs one store-to-load latency (~0.5 us measured);
//   * a layer's down weights and the next layer's router rows do not depend on h / x: they are requested as soon as
//     the top-k is known and sit in registers while gate/up streams, so the layer's bytes are in flight together;
//   * each wait is bounded by a wall-clock deadline and a shared abort flag, so a launch always ends; a timed-out
//     launch leaves a nonzero status in the workspace header.
//
// Per layer l (x_0 is the input, x_{l+1} = x_l + moe_l(x_l), f16 between layers as the reference's activations):
//   A. x_l -> LDS (raw f16 and prepared units); workgroups owning router rows compute their logits (the router
//      weight rows came in during the previous layer) and publish them;
//   B. every workgroup polls the E (+1 shared gate) logits and ranks them itself (ties to the lower index);
//   C. loads: this workgroup's gate/up rows (a contiguous range of the k I + Is pair-rows), its down rows (a range
//      of output rows, all slots), the next layer's router rows;
//   D. gate/up dots + SwiGLU, h published as f16 pairs;
//   E. all of h polled into LDS as prepared units;
//   F. down dots weighted by the router scores (the shared expert by sigmoid of its gate logit), + x_l, published
//      as x_{l+1} (the last layer writes the output).
//
// Router logit order (restated by the test oracle bit for bit): thread t of 512 holds elements [C t, C t + C),
// C = H / 512, and sums x_i w_i over them in element order (f16 x f16 products are exact in fp32, so each step
// rounds once); the 512 partials are added as a balanced binary tree in thread order.
#include <algorithm>

#include "lmoe_common.h"

namespace lmoe {

namespace stk {

constexpr int NT = 512;  // threads a workgroup
constexpr int NW = NT / 64;
constexpr int KMAX = 16;    // routed experts a token
constexpr int EMAX = 512;   // routed experts
constexpr int RRMAX = 3;    // router rows a workgroup
constexpr int HWMAX = 12;   // h words a thread (k I + Is <= 2 * 512 * 12)
constexpr int NPMAX2 = 64;  // pair-row pairs a workgroup (np <= 128)
constexpr int NRMAX2 = 32;  // output row pairs a workgroup (nr <= 64)
constexpr long long kTimeoutTicks = 20000000;  // 0.2 s of the 100 MHz wall clock a wait

// the small-scratch region (dword offsets)
constexpr int MI_PICK = 0, MI_PSC = KMAX, MI_PRAW = 2 * KMAX, MI_RED = 3 * KMAX, MI_SK = MI_RED + 8 * RRMAX,
              MI_SI = MI_SK + 8 * KMAX, MI_HLOC = MI_SI + 8 * KMAX, MI_XOUT = MI_HLOC + NPMAX2,
              MI_ROWDOT = MI_XOUT + 2 * NRMAX2, MI_END = MI_ROWDOT + 4 * NPMAX2;

struct Args {
  int L, H, E, k, I, Is, norm;
  const uint8_t *const *wg;  // [L] -> [E, I, 36 H / 64]
  const uint8_t *const *wu;
  const uint8_t *const *wd;  // [L] -> [E, H, 36 I / 64]
  const uint16_t *const *wr;   // [L] -> [E, H] f16
  const uint16_t *const *wsg;  // [L] -> [H] f16 (shared expert's gate), or null without a shared expert
  const uint8_t *const *sg;    // [L] -> [Is, 36 H / 64]
  const uint8_t *const *su;
  const uint8_t *const *sd;  // [L] -> [H, 36 Is / 64]
  const uint16_t *x0;        // [H] f16
  uint16_t *out;             // [H] f16
  uint32_t *hdr;             // workspace header: [0] epoch of the last launch, [1] status
  uint64_t *xw;              // [L - 1][H / 2] x_1 .. x_{L-1} as f16 pairs
  uint64_t *lw;              // [L][E + shared] logits
  uint64_t *hw;              // [L][(k I + Is) / 2] h as f16 pairs
  float *y;                  // [L][H] the layer's MoE output (f32, before the residual), or null
  uint32_t *ids;             // [L][k] or null
  float *scores;             // [L][k] or null
  // LDS byte offsets
  int o_xraw, o_xprep, o_keys, o_misc, o_hprep, o_stage;
};

__device__ __forceinline__ uint64_t ld_word(const uint64_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_word(uint64_t *p, uint32_t payload, uint32_t ep) {
  __hip_atomic_store(p, uint64_t(payload) | (uint64_t(ep) << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_status(const uint32_t *hdr) {
  return __hip_atomic_load(hdr + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void set_status(uint32_t *hdr, uint32_t code) {
  __hip_atomic_store(hdr + 1, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// This thread's words src[tid + NT a] (a < NA, index < n) into v[a], polled until each carries epoch ep. False when
// the deadline passes (the status is then set) or another workgroup has set the status.
template <int NA>
__device__ __forceinline__ bool poll_words(const uint64_t *src, int n, uint32_t ep, uint64_t *v, uint32_t *hdr,
                                           int tid) {
#pragma unroll
  for (int a = 0; a < NA; ++a) v[a] = ld_word(src + min(tid + NT * a, n - 1));
  const long long t0 = wall_clock64();
  for (int it = 0;; ++it) {
    uint32_t pend = 0;
#pragma unroll
    for (int a = 0; a < NA; ++a)
      if (tid + NT * a < n && uint32_t(v[a] >> 32) != ep) pend |= 1u << a;
    if (!pend) return true;
    __builtin_amdgcn_s_sleep(2);
    if ((it & 15) == 15) {
      if (ld_status(hdr)) return false;
      if (wall_clock64() - t0 > kTimeoutTicks) {
        set_status(hdr, 1u);
        return false;
      }
    }
#pragma unroll
    for (int a = 0; a < NA; ++a)
      if ((pend >> a) & 1u) v[a] = ld_word(src + tid + NT * a);
  }
}

// a balanced binary tree over the workgroup's 512 values, in thread order; every thread gets the total.
// red: NW floats of LDS. Two barriers.
__device__ __forceinline__ float block_tree(float v, float *red, int tid) {
  v = wave_sum(v);
  const int lane = tid & 63, wave = tid >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  return ((red[0] + red[1]) + (red[2] + red[3])) + ((red[4] + red[5]) + (red[6] + red[7]));
}

// 16 / 8 bytes from global memory with the nontemporal hint; the address-space cast keeps the compiler from
// falling back to flat loads for pointers picked from tables
__device__ __forceinline__ u32x4 ldg_nt4(const void *p) {
  return __builtin_nontemporal_load(
      (const __attribute__((address_space(1))) u32x4 *)(reinterpret_cast<uintptr_t>(p)));
}
__device__ __forceinline__ u32x2 ldg_nt2(const void *p) {
  return __builtin_nontemporal_load(
      (const __attribute__((address_space(1))) u32x2 *)(reinterpret_cast<uintptr_t>(p)));
}

// entry l of a device table of pointers, read through the constant address space (scalar loads: the tables do not
// change during a launch)
__device__ __forceinline__ const uint8_t *table_at(const void *const *tab, int l) {
  const __attribute__((address_space(4))) uint64_t *t =
      (const __attribute__((address_space(4))) uint64_t *)(reinterpret_cast<uintptr_t>(tab));
  return reinterpret_cast<const uint8_t *>(uintptr_t(t[l]));
}


__device__ __forceinline__ float f16f(uint32_t bits16) {
  return float(__builtin_bit_cast(_Float16, uint16_t(bits16)));
}

// (ids, scores) of the top k of the E logits in LDS (vals), into pick / psc (k entries, best first).
// ck: 512 u64, cnt: 2048 u32, surv: 128 u64, praw: KMAX floats, red: 8 floats of LDS scratch. All threads; ends
// with a barrier. E <= 128: each of the 512 threads counts, for candidate t % 128, the candidates above it among one
// quarter; the four quarter counts are its rank. E <= 512: the same over chunks of 64 (the top k of each chunk
// survive), then over the survivors.
__device__ __forceinline__ void topk_block(const float *vals, int E, int k, int norm, uint32_t *pick, float *psc,
                                           float *praw, uint64_t *ck, uint32_t *cnt, uint64_t *surv, float *red,
                                           int tid) {
  const uint64_t mine_key = tid < E ? (uint64_t(logit_key(vals[tid])) << 32) | (0xFFFFFFFFu - uint32_t(tid)) : 0u;
  ck[tid] = mine_key;
  if (E > 128 && tid < 128) surv[tid] = 0u;
  __syncthreads();
  const uint64_t *set = ck;
  int nset = E;
  if (E > 128) {
    // stage 1: rank inside the 64-candidate chunk; the chunk's best k survive, at surv[chunk k + rank]
    const int c = count_above<32>(ck, tid & ~63, mine_key);
    if (tid < E && c < k) surv[(tid >> 6) * k + c] = mine_key;
    __syncthreads();
    set = surv;
    nset = ((E + 63) >> 6) * k;
  }
  // rank among the set (<= 128 entries, padded with zeros): thread t holds entries g, g + 32, g + 64, g + 96
  // (g = t % 32) and counts the entries above each among the 8 entries [8 q, 8 q + 8) (q = t / 32): 4 LDS reads and
  // 32 compares a thread; entry i's rank is the sum of its 16 counts
  {
    typedef uint64_t u64x2 __attribute__((ext_vector_type(2)));
    const int g = tid & 31, q = tid >> 5;
    const u64x2 *p8 = reinterpret_cast<const u64x2 *>(set + 8 * q);
    uint64_t o[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u64x2 v = p8[j];
      o[2 * j] = v.x;
      o[2 * j + 1] = v.y;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint64_t me = set[g + 32 * i];
      int c = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) c += o[j] > me ? 1 : 0;
      cnt[(g + 32 * i) * 16 + q] = uint32_t(c);
    }
  }
  __syncthreads();
  if (tid < 128 && tid < nset && set[tid] != 0u) {
    const u32x4 *c4 = reinterpret_cast<const u32x4 *>(cnt + 16 * tid);
    int r = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u32x4 v = c4[j];
      r += int(v.x + v.y + v.z + v.w);
    }
    if (r < k) pick[r] = 0xFFFFFFFFu - uint32_t(set[tid]);
  }
  __syncthreads();
  // softmax over the E logits (max subtracted), the picks' probabilities, renormalised in rank order when norm
  const float m = vals[pick[0]];
  const float term = tid < E ? __expf(vals[tid] - m) : 0.0f;
  const float s = block_tree(term, red, tid);
  float mine = 0.0f;
  if (tid < k) {
    mine = __expf(vals[pick[tid]] - m) / s;
    praw[tid] = mine;
  }
  __syncthreads();
  if (tid < k) {
    float tot = 0.0f;  // the k probabilities summed in rank order
    for (int r = 0; r < k; ++r) tot += praw[r];
    psc[tid] = norm ? mine / tot : mine;
  }
  __syncthreads();
}

}  // namespace stk

// TQ: block type of every projection; HH: hidden size (2048 or 4096); NCG / NCD: 16-byte gate/up and down chunks a
// thread a layer (the host checks the shapes fit).
template <int TQ, int HH, int NCG, int NCD>
__global__ void __launch_bounds__(stk::NT, 1) k_stack(stk::Args a) {
  using namespace stk;
  constexpr int P = HH / 64;         // units of an x row
  constexpr int RBH = 36 * P;        // bytes of a gate / up row
  constexpr int CPR = RBH / 16;      // 16-byte chunks of a gate / up row
  constexpr int C = HH / NT;         // x elements a thread (router)
  constexpr int CW = C / 2;          // x words a thread
  constexpr int GP = NT / P;         // lane groups (one pair-row each a pass)
  constexpr int HT = TQ == LMOE_Q4_K ? 32 : 16;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid0 = threadIdx.x;
  const int b = blockIdx.x, nb = gridDim.x;
  const int L = a.L, E = a.E, k = a.k, I = a.I, Is = a.Is;
  const bool shared = Is > 0;
  const int Etot = E + (shared ? 1 : 0);
  const int S = k + (shared ? 1 : 0);
  const int PI = I / 64, PIs = Is / 64;
  const int RBI = 36 * PI, RBIs = 36 * PIs;
  const int NPR = k * I + Is;          // pair-rows (h values) a layer
  const int Utot = k * PI + PIs;       // h units
  const int p0 = 2 * int((long long)b * (NPR / 2) / nb), p1 = 2 * int((long long)(b + 1) * (NPR / 2) / nb);
  const int np = p1 - p0;
  const int n0 = 2 * int((long long)b * (HH / 2) / nb), n1 = 2 * int((long long)(b + 1) * (HH / 2) / nb);
  const int nr = n1 - n0;
  const int nrr = b < Etot ? (Etot - 1 - b) / nb + 1 : 0;  // router rows e = b + nb i
  const int RPB = 2 * (k * RBI + RBIs);                     // down stage bytes of a row pair
  const int ngc = np * 2 * CPR, ndc = (nr / 2) * (RPB / 16);

  uint16_t *xraw = reinterpret_cast<uint16_t *>(lds + a.o_xraw);
  uint32_t *xprep = reinterpret_cast<uint32_t *>(lds + a.o_xprep);
  float *vals = reinterpret_cast<float *>(lds + a.o_keys);                            // EMAX + 16 logits
  uint64_t *ckeys = reinterpret_cast<uint64_t *>(lds + a.o_keys + 4 * (EMAX + 16));   // NT composite keys
  uint32_t *cnt = reinterpret_cast<uint32_t *>(lds + a.o_keys + 4 * (EMAX + 16) + 8 * NT);  // 2048 counts
  uint32_t *misc = reinterpret_cast<uint32_t *>(lds + a.o_misc);
  uint32_t *pick = misc + MI_PICK;
  float *psc = reinterpret_cast<float *>(misc + MI_PSC);
  float *praw = reinterpret_cast<float *>(misc + MI_PRAW);
  float *red = reinterpret_cast<float *>(misc + MI_RED);
  uint64_t *surv = reinterpret_cast<uint64_t *>(misc + MI_SK);  // 8 KMAX survivors (MI_SK..MI_SI + 8 KMAX)
  uint16_t *hloc = reinterpret_cast<uint16_t *>(misc + MI_HLOC);  // np (<= 2 NPMAX2) f16
  float *xout = reinterpret_cast<float *>(misc + MI_XOUT);        // nr (<= 2 NRMAX2) f32
  float *rowdot = reinterpret_cast<float *>(misc + MI_ROWDOT);    // 2 np (<= 4 NPMAX2) f32
  uint32_t *hprep = reinterpret_cast<uint32_t *>(lds + a.o_hprep);
  uint8_t *stage = lds + a.o_stage;

  // a launch after a timed-out one does nothing until the workspace is cleared (its words may carry this epoch)
  if (a.hdr[1] != 0u) return;
  const uint32_t ep = a.hdr[0] + 1u;

  // router rows of layer 0
  uint32_t wrr[RRMAX][CW];
  auto load_router = [&](int l, int tid) {
#pragma unroll
    for (int i = 0; i < RRMAX; ++i) {
      const int e = min(b + nb * i, Etot - 1);
      const uint16_t *row = e < E ? reinterpret_cast<const uint16_t *>(table_at(
                                          reinterpret_cast<const void *const *>(a.wr), l)) + size_t(e) * HH
                                    : reinterpret_cast<const uint16_t *>(
                                          table_at(reinterpret_cast<const void *const *>(a.wsg), l));
      if (CW == 2) {
        const u32x2 v = ldg_nt2(row + 4 * tid);
        wrr[i][0] = v.x;
        wrr[i][CW - 1] = v.y;
      } else {
        const u32x4 v = ldg_nt4(row + 8 * tid);
        wrr[i][0] = v.x;
        wrr[i][1 % CW] = v.y;
        wrr[i][2 % CW] = v.z;
        wrr[i][3 % CW] = v.w;
      }
    }
  };
  if (nrr > 0) load_router(0, tid0);

  // Per-thread address tables, the same every layer: gate/up chunk q is byte gofs[q] of the expert matrix picked by
  // slot gsel[q] >> 1 (gate when gsel[q] & 1 is 0, up when 1); down chunk q is byte dofs[q] of slot dsel[q]'s down
  // matrix; h word q's two values go to halfwords emap[q] & 0xFFFF and emap[q] >> 16 of the prepared h units.
  uint32_t gofs[NCG], gsel[NCG], dofs[NCD], dsel[NCD], emap[HWMAX];
#pragma unroll
  for (int q = 0; q < NCG; ++q) {
    const int c = min(tid0 + NT * q, ngc - 1);
    const int i = c / (2 * CPR), m = (c / CPR) & 1, cc = c - (c / CPR) * CPR;
    const int p = p0 + i;
    const int sl = p < k * I ? p / I : k, r = p - sl * I;
    gofs[q] = uint32_t(r * RBH + 16 * cc);
    gsel[q] = uint32_t(2 * sl + m);
  }
  const int kc = k * (2 * RBI / 16);  // chunks of the routed part of a row pair
  const int rpc = RPB / 16;
#pragma unroll
  for (int q = 0; q < NCD; ++q) {
    const int c = min(tid0 + NT * q, ndc - 1);
    const int rp = c / rpc, cq = c - rp * rpc;
    const int n = n0 + 2 * rp;
    if (cq < kc) {
      const int sl = cq / (2 * RBI / 16);
      dofs[q] = uint32_t(n * RBI + 16 * (cq - sl * (2 * RBI / 16)));
      dsel[q] = uint32_t(sl);
    } else {
      dofs[q] = uint32_t(n * RBIs + 16 * (cq - kc));
      dsel[q] = uint32_t(k);
    }
  }
#pragma unroll
  for (int q = 0; q < HWMAX; ++q) {
    uint32_t t2 = 0;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int j = min(2 * (tid0 + NT * q) + hh, NPR - 1);
      const int sl = j < k * I ? j / I : k, r = j - sl * I;
      int dw, half;
      xslot(r & 63, HT, &dw, &half);
      t2 |= uint32_t(2 * ((sl * PI + (r >> 6)) * XS + dw) + half) << (16 * hh);
    }
    emap[q] = t2;
  }

  // this layer's expert matrices (scalar loads, one layer ahead of their use)
  auto tab = [&](const uint8_t *const *t, int l) {
    return t ? table_at(reinterpret_cast<const void *const *>(t), l) : nullptr;
  };
  const uint8_t *nwg = tab(a.wg, 0), *nwu = tab(a.wu, 0), *nwd = tab(a.wd, 0);
  const uint8_t *nsg = shared ? tab(a.sg, 0) : nullptr, *nsu = shared ? tab(a.su, 0) : nullptr;
  const uint8_t *nsd = shared ? tab(a.sd, 0) : nullptr;

  for (int l = 0; l < L; ++l) {
    const int tid = opaque(tid0), lane = tid & 63, wave = tid >> 6;
    const uint8_t *wgl = nwg, *wul = nwu, *wdl = nwd, *sgl = nsg, *sul = nsu, *sdl = nsd;
    if (l + 1 < L) {
      nwg = tab(a.wg, l + 1), nwu = tab(a.wu, l + 1), nwd = tab(a.wd, l + 1);
      if (shared) nsg = tab(a.sg, l + 1), nsu = tab(a.su, l + 1), nsd = tab(a.sd, l + 1);
    }
#pragma unroll
    for (int q = 0; q < NCG; ++q) gofs[q] = opaque(gofs[q]), gsel[q] = opaque(gsel[q]);
#pragma unroll
    for (int q = 0; q < NCD; ++q) dofs[q] = opaque(dofs[q]), dsel[q] = opaque(dsel[q]);
#pragma unroll
    for (int q = 0; q < HWMAX; ++q) emap[q] = opaque(emap[q]);
    // ---- A. x_l into LDS; router logits ----------------------------------------------------------------------
    uint32_t xv[CW];
    if (l == 0) {
#pragma unroll
      for (int q = 0; q < CW; ++q) xv[q] = reinterpret_cast<const uint32_t *>(a.x0)[CW * tid + q];
    } else {
      uint64_t w[CW];
      const uint64_t *src = a.xw + size_t(l - 1) * (HH / 2) + CW * tid;
#pragma unroll
      for (int q = 0; q < CW; ++q) w[q] = ld_word(src + q);
      // poll the CW consecutive words of this thread
      const long long t0 = wall_clock64();
      bool ok = true;
      for (int it = 0;; ++it) {
        bool done = true;
#pragma unroll
        for (int q = 0; q < CW; ++q) done = done && uint32_t(w[q] >> 32) == ep;
        if (done) break;
        __builtin_amdgcn_s_sleep(2);
        if ((it & 15) == 15) {
          if (ld_status(a.hdr)) { ok = false; break; }
          if (wall_clock64() - t0 > kTimeoutTicks) { set_status(a.hdr, 1u); ok = false; break; }
        }
#pragma unroll
        for (int q = 0; q < CW; ++q)
          if (uint32_t(w[q] >> 32) != ep) w[q] = ld_word(src + q);
      }
      if (__syncthreads_or(!ok)) return;
#pragma unroll
      for (int q = 0; q < CW; ++q) xv[q] = uint32_t(w[q]);
    }
#pragma unroll
    for (int q = 0; q < CW; ++q) reinterpret_cast<uint32_t *>(xraw)[CW * tid + q] = xv[q];
    if (nrr > 0) {
      // this thread's elements [C tid, C tid + C) in order; f16 x f16 products are exact, one rounding a step
      float part[RRMAX];
#pragma unroll
      for (int i = 0; i < RRMAX; ++i) {
        float acc = 0.0f;
#pragma unroll
        for (int q = 0; q < CW; ++q) {
          const float x0 = f16f(xv[q] & 0xFFFFu), x1 = f16f(xv[q] >> 16);
          const float w0 = f16f(wrr[i][q] & 0xFFFFu), w1 = f16f(wrr[i][q] >> 16);
          acc = q == 0 ? x0 * w0 : fmaf(x0, w0, acc);
          acc = fmaf(x1, w1, acc);
        }
        part[i] = wave_sum(acc);
      }
      if (lane == 0) {
#pragma unroll
        for (int i = 0; i < RRMAX; ++i) red[8 * i + wave] = part[i];
      }
    }
    __syncthreads();
    if (tid < nrr) {
      const float *r8 = red + 8 * tid;
      const float lg = ((r8[0] + r8[1]) + (r8[2] + r8[3])) + ((r8[4] + r8[5]) + (r8[6] + r8[7]));
      st_word(a.lw + size_t(l) * Etot + b + nb * tid, __float_as_uint(lg), ep);
    }
    // prepared x units (pairs in nibble order + half sums), then this lane's unit into registers
    for (int idx = tid; idx < 36 * P; idx += NT) {
      const int p = idx / 36, dw = idx - p * 36;
      xprep[idx] = prep_dword<TQ>([&](int i) { return f16f(xraw[i]); }, p, dw);
    }

    // ---- B. logits -> top-k ------------------------------------------------------------------------------
    {
      uint64_t w[2];
      const bool ok = poll_words<2>(a.lw + size_t(l) * Etot, Etot, ep, w, a.hdr, tid);
      if (__syncthreads_or(!ok)) return;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int e = tid + NT * q;
        if (e < Etot) vals[e] = __uint_as_float(uint32_t(w[q]));
      }
    }
    __syncthreads();
    stk::topk_block(vals, E, k, a.norm, pick, psc, praw, ckeys, cnt, surv, red, tid);
    if (b == 0 && tid < k) {
      if (a.ids) a.ids[size_t(l) * k + tid] = pick[tid];
      if (a.scores) a.scores[size_t(l) * k + tid] = psc[tid];
    }

    // ---- C. loads: gate/up rows, down rows, next router rows ----------------------------------------------
    const size_t gstride = size_t(I) * RBH, dstride = size_t(HH) * RBI;
    u32x4 gv[NCG];
#pragma unroll
    for (int q = 0; q < NCG; ++q) {
      const uint32_t sl = gsel[q] >> 1, m = gsel[q] & 1u;
      const uint32_t e = pick[min(sl, uint32_t(k - 1))];  // read for every chunk: no branch around the LDS read
      const uint8_t *rb = m ? wul : wgl, *sb = m ? sul : sgl;
      const uint8_t *base = sl < uint32_t(k) ? rb + size_t(e) * gstride : sb;
      gv[q] = ldg_nt4(base + gofs[q]);
    }
    asm volatile("" ::: "memory");
    u32x4 dv[NCD];
#pragma unroll
    for (int q = 0; q < NCD; ++q) {
      const uint32_t sl = dsel[q];
      const uint32_t e = pick[min(sl, uint32_t(k - 1))];
      const uint8_t *base = sl < uint32_t(k) ? wdl + size_t(e) * dstride : sdl;
      dv[q] = ldg_nt4(base + dofs[q]);
    }
    asm volatile("" ::: "memory");
    if (nrr > 0 && l + 1 < L) load_router(l + 1, tid);

    // ---- D. gate/up + SwiGLU, h published ----------------------------------------------------------------
    // The stage holds 2 np rows (pair i: gate row 2 i, up row 2 i + 1). Passes of NT / P rows: each stores the chunks
    // its rows need that are not in LDS yet (so it waits only for the earlier loads) and dots one row a lane group,
    // while the later rows' loads are still in flight; the row dots go to LDS, SwiGLU follows.
    {
      const int g = tid / P, p = tid - g * P;
      uint32_t xu[32];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const u32x4 v = reinterpret_cast<const u32x4 *>(xprep)[9 * p + i];
        xu[4 * i] = v.x;
        xu[4 * i + 1] = v.y;
        xu[4 * i + 2] = v.z;
        xu[4 * i + 3] = v.w;
      }
      const u32x4 sv = reinterpret_cast<const u32x4 *>(xprep)[9 * p + 8];
      const float sx0 = __uint_as_float(sv.x), sx1 = __uint_as_float(sv.y);
      const uint32_t *st = reinterpret_cast<const uint32_t *>(stage);
      u32x4 *st4 = reinterpret_cast<u32x4 *>(stage);
      const int R2 = 2 * np;
      int have = 0;  // chunks in LDS
      for (int r0 = 0; r0 < R2; r0 += GP) {
        const int lim = min(ngc, (r0 + GP) * CPR);
#pragma unroll
        for (int q = 0; q < NCG; ++q) {
          const int c = tid + NT * q;
          if (c >= have && c < lim) st4[c] = gv[q];
        }
        have = lim;
        __syncthreads();
        const int r = min(r0 + g, R2 - 1);
        const float d = group_sum<P>(row_unit_dot_r<TQ>(st + r * (RBH / 4), p, xu, sx0, sx1));
        if (p == 0 && r0 + g < R2) rowdot[r0 + g] = d;
      }
    }
    __syncthreads();
    if (tid < np) hloc[tid] = __builtin_bit_cast(uint16_t, _Float16(silu_mul(rowdot[2 * tid], rowdot[2 * tid + 1])));
    __syncthreads();
    if (tid < np / 2) {
      const uint32_t pr = uint32_t(hloc[2 * tid]) | (uint32_t(hloc[2 * tid + 1]) << 16);
      st_word(a.hw + size_t(l) * (NPR / 2) + p0 / 2 + tid, pr, ep);
    }

    // ---- E. h -> LDS as prepared units ------------------------------------------------------------------------
    {
      uint64_t w[HWMAX];
      const bool ok = poll_words<HWMAX>(a.hw + size_t(l) * (NPR / 2), NPR / 2, ep, w, a.hdr, tid);
      if (__syncthreads_or(!ok)) return;
      uint16_t *hp16 = reinterpret_cast<uint16_t *>(hprep);
#pragma unroll
      for (int q = 0; q < HWMAX; ++q) {
        if (tid + NT * q >= NPR / 2) continue;
        hp16[emap[q] & 0xFFFFu] = uint16_t(uint32_t(w[q]));
        hp16[emap[q] >> 16] = uint16_t(uint32_t(w[q]) >> 16);
      }
    }
    __syncthreads();
    // a unit's sums over its first / last 32 values (dwords 32, 33)
    for (int hu = tid; hu < 2 * Utot; hu += NT) {
      const int U = hu >> 1, half = hu & 1;
      const uint32_t *u = hprep + U * XS;
      float s = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const uint32_t w = TQ == LMOE_Q4_K ? u[2 * i + half] : u[16 * half + i];
        s += half_lo(w) + half_hi(w);
      }
      hprep[U * XS + 32 + half] = __builtin_bit_cast(uint32_t, s);
    }
    // the down weights into the stage (gate/up's reads of it ended at the barrier above)
    {
      u32x4 *st4 = reinterpret_cast<u32x4 *>(stage);
#pragma unroll
      for (int q = 0; q < NCD; ++q) {
        const int c = tid + NT * q;
        if (c < ndc) st4[c] = dv[q];
      }
    }
    __syncthreads();

    // ---- F. down + weighted combine + residual -------------------------------------------------------------
    {
      const float gsh = shared ? sigmoidf_(vals[E]) : 0.0f;
      const uint32_t *st = reinterpret_cast<const uint32_t *>(stage);
      for (int rr = wave; rr < nr; rr += NW) {
        const int rp = rr >> 1, odd = rr & 1;
        float acc = 0.0f;
        for (int u0 = 0; u0 < Utot; u0 += 64) {
          const int u = min(u0 + lane, Utot - 1);
          int s, j;
          if (u < k * PI) {
            s = u / PI;
            j = u - s * PI;
          } else {
            s = k;
            j = u - k * PI;
          }
          const int rb = s < k ? RBI : RBIs;
          const uint32_t *row = st + (rp * RPB + s * 2 * RBI + odd * rb) / 4;
          const uint32_t *hu = hprep + u * XS;
          uint32_t hv[32];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const u32x4 v = reinterpret_cast<const u32x4 *>(hu)[i];
            hv[4 * i] = v.x;
            hv[4 * i + 1] = v.y;
            hv[4 * i + 2] = v.z;
            hv[4 * i + 3] = v.w;
          }
          const u32x4 sv = reinterpret_cast<const u32x4 *>(hu)[8];
          const float d = row_unit_dot_r<TQ>(row, j, hv, __uint_as_float(sv.x), __uint_as_float(sv.y));
          const float wt = s < k ? psc[s] : gsh;
          acc = (u0 + lane < Utot) ? fmaf(wt, d, acc) : acc;
        }
        acc = wave_sum(acc);
        if (lane == 0) {
          const int n = n0 + rr;
          if (a.y) a.y[size_t(l) * HH + n] = acc;
          xout[rr] = f16f(xraw[n]) + acc;
        }
      }
    }
    __syncthreads();
    if (tid < nr / 2) {
      const uint32_t pr = uint32_t(__builtin_bit_cast(uint16_t, _Float16(xout[2 * tid]))) |
                          (uint32_t(__builtin_bit_cast(uint16_t, _Float16(xout[2 * tid + 1]))) << 16);
      if (l + 1 < L)
        st_word(a.xw + size_t(l) * (HH / 2) + n0 / 2 + tid, pr, ep);
      else
        reinterpret_cast<uint32_t *>(a.out)[n0 / 2 + tid] = pr;
    }
  }
  // every workgroup read the epoch before it published its first word, and workgroup 0 has seen every workgroup's
  // last h: the next launch may take the next epoch
  if (b == 0 && tid0 == 0) a.hdr[0] = ep;
}

// ---- host ---------------------------------------------------------------------------------------------------------

namespace {

struct Layout {
  int lds;
  int o_xraw, o_xprep, o_keys, o_misc, o_hprep, o_stage;
  int ncg, ncd;  // chunks a thread the largest workgroup needs
};

Layout stack_layout(int H, int E, int k, int I, int Is, int nb) {
  Layout s{};
  const int P = H / 64;
  const int NPR = k * I + Is;
  const int Utot = (k * I + Is) / 64;
  int npmax = 0, nrmax = 0;
  for (int b = 0; b < nb; ++b) {
    const int p0 = 2 * int((long long)b * (NPR / 2) / nb), p1 = 2 * int((long long)(b + 1) * (NPR / 2) / nb);
    const int n0 = 2 * int((long long)b * (H / 2) / nb), n1 = 2 * int((long long)(b + 1) * (H / 2) / nb);
    npmax = std::max(npmax, p1 - p0);
    nrmax = std::max(nrmax, n1 - n0);
  }
  const int RBH = 36 * P, RBI = 36 * (I / 64), RBIs = 36 * (Is / 64);
  const int gbytes = npmax * 2 * RBH;
  const int dbytes = (nrmax / 2) * 2 * (k * RBI + RBIs);
  s.ncg = (gbytes / 16 + stk::NT - 1) / stk::NT;
  s.ncd = (dbytes / 16 + stk::NT - 1) / stk::NT;
  int o = 0;
  auto take = [&](int bytes) {
    const int at = o;
    o += (bytes + 15) & ~15;
    return at;
  };
  s.o_xraw = take(2 * H);
  s.o_xprep = take(P * XS * 4);
  s.o_keys = take(4 * (stk::EMAX + 16) + 8 * stk::NT + 4 * 2048);
  s.o_misc = take(4 * stk::MI_END);
  s.o_hprep = take(Utot * XS * 4);
  s.o_stage = take(std::max(gbytes, dbytes));
  s.lds = o;
  (void)E;
  return s;
}

int g_num_cus = 0;

}  // namespace

template <int TQ, int HH, int NCG, int NCD>
static int launch_stack(stk::Args a, int lds, int nb, hipStream_t st) {
  auto kern = k_stack<TQ, HH, NCG, NCD>;
  if (int rc = allow_lds(kern, size_t(lds), "lmoe_stack_decode")) return rc;
  int per_cu = 0;
  hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, stk::NT, lds);
  if (e != hipSuccess) return hip_fail(e, "lmoe_stack_decode: occupancy");
  LMOE_REQUIRE(per_cu >= 1, LMOE_ESHAPE, "lmoe_stack_decode: the kernel does not fit a CU (%d bytes of LDS)", lds);
  void *args[] = {&a};
  e = hipLaunchCooperativeKernel(reinterpret_cast<const void *>(kern), dim3(nb), dim3(stk::NT), args,
                                 uint32_t(lds), st);
  if (e != hipSuccess) return hip_fail(e, "lmoe_stack_decode");
  return 0;
}

}  // namespace lmoe

using namespace lmoe;

extern "C" size_t lmoe_stack_workspace_bytes(int L, int H, int E, int k, int I, int Is) {
  if (L <= 0 || H <= 0 || E <= 0 || k <= 0 || I <= 0 || Is < 0) return 0;
  const size_t etot = size_t(E) + (Is > 0 ? 1 : 0);
  return 256 + 8 * (size_t(L > 1 ? L - 1 : 0) * (H / 2) + size_t(L) * etot + size_t(L) * ((size_t(k) * I + Is) / 2));
}

extern "C" int lmoe_stack_decode(int L, int H, int E, int k, int I, int Is, int qtype, int norm,
                                 const void *const *wg, const void *const *wu, const void *const *wd,
                                 const void *const *wr, const void *const *wsg, const void *const *sg,
                                 const void *const *su, const void *const *sd, const void *x, void *out,
                                 void *workspace, float *y, uint32_t *ids, float *scores, void *stream) {
  LMOE_REQUIRE(L >= 1, LMOE_ESHAPE, "lmoe_stack_decode: %d layers", L);
  LMOE_REQUIRE(H == 2048 || H == 4096, LMOE_ESHAPE, "lmoe_stack_decode: hidden %d (2048 or 4096)", H);
  LMOE_REQUIRE(E >= 1 && E <= stk::EMAX, LMOE_ESHAPE, "lmoe_stack_decode: %d experts (1..%d)", E, stk::EMAX);
  LMOE_REQUIRE(k >= 1 && k <= stk::KMAX && k <= E, LMOE_ESHAPE, "lmoe_stack_decode: top-%d of %d", k, E);
  LMOE_REQUIRE(I > 0 && I % 128 == 0 && Is >= 0 && Is % 128 == 0, LMOE_ESHAPE,
               "lmoe_stack_decode: intermediate %d / shared %d must be multiples of 128", I, Is);
  LMOE_REQUIRE(qtype_ok(qtype), LMOE_ETYPE, "lmoe_stack_decode: block type %d (Q4_0 or Q4_K)", qtype);
  LMOE_REQUIRE(qtype != LMOE_Q4_K || (I % 256 == 0 && Is % 256 == 0), LMOE_ESHAPE,
               "lmoe_stack_decode: Q4_K rows of %d / %d weights", I, Is);
  LMOE_REQUIRE(wg && wu && wd && wr && x && out && workspace, LMOE_EINVAL, "lmoe_stack_decode: null pointer");
  LMOE_REQUIRE(Is == 0 || (wsg && sg && su && sd), LMOE_EINVAL, "lmoe_stack_decode: shared expert pointers");
  LMOE_REQUIRE(aligned16(workspace) && aligned4(x) && aligned4(out), LMOE_EALIGN, "lmoe_stack_decode: alignment");
  LMOE_REQUIRE((size_t(k) * I + Is) / 2 <= size_t(stk::NT) * stk::HWMAX, LMOE_ESHAPE,
               "lmoe_stack_decode: %d h values a layer (at most %d)", k * I + Is, 2 * stk::NT * stk::HWMAX);
  if (g_num_cus == 0) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&g_num_cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return hip_fail(e, "lmoe_stack_decode: device query");
  }
  const int nb = g_num_cus;
  LMOE_REQUIRE(E + (Is > 0 ? 1 : 0) <= nb * stk::RRMAX, LMOE_ESHAPE, "lmoe_stack_decode: %d router rows", E);
  const Layout lay = stack_layout(H, E, k, I, Is, nb);
  LMOE_REQUIRE(lay.lds <= 160 * 1024, LMOE_ESHAPE, "lmoe_stack_decode: %d bytes of LDS", lay.lds);
  const int npw = ((k * I + Is) / 2 + nb - 1) / nb, nrw = (H / 2 + nb - 1) / nb;  // pairs a workgroup at most
  LMOE_REQUIRE(npw <= stk::NPMAX2 && nrw <= stk::NRMAX2 && (k * I + Is) / 2 >= nb && H / 2 >= nb, LMOE_ESHAPE,
               "lmoe_stack_decode: %d h pairs and %d output-row pairs over %d workgroups", (k * I + Is) / 2, H / 2,
               nb);
  stk::Args a{};
  a.L = L, a.H = H, a.E = E, a.k = k, a.I = I, a.Is = Is, a.norm = norm;
  a.wg = reinterpret_cast<const uint8_t *const *>(wg);
  a.wu = reinterpret_cast<const uint8_t *const *>(wu);
  a.wd = reinterpret_cast<const uint8_t *const *>(wd);
  a.wr = reinterpret_cast<const uint16_t *const *>(wr);
  a.wsg = reinterpret_cast<const uint16_t *const *>(wsg);
  a.sg = reinterpret_cast<const uint8_t *const *>(sg);
  a.su = reinterpret_cast<const uint8_t *const *>(su);
  a.sd = reinterpret_cast<const uint8_t *const *>(sd);
  a.x0 = static_cast<const uint16_t *>(x);
  a.out = static_cast<uint16_t *>(out);
  uint8_t *ws = static_cast<uint8_t *>(workspace);
  a.hdr = reinterpret_cast<uint32_t *>(ws);
  const size_t etot = size_t(E) + (Is > 0 ? 1 : 0);
  a.xw = reinterpret_cast<uint64_t *>(ws + 256);
  a.lw = a.xw + size_t(L > 1 ? L - 1 : 0) * (H / 2);
  a.hw = a.lw + size_t(L) * etot;
  a.y = y, a.ids = ids, a.scores = scores;
  a.o_xraw = lay.o_xraw, a.o_xprep = lay.o_xprep, a.o_keys = lay.o_keys, a.o_misc = lay.o_misc;
  a.o_hprep = lay.o_hprep, a.o_stage = lay.o_stage;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool small = lay.ncg <= 8 && lay.ncd <= 4;
  LMOE_REQUIRE(lay.ncg <= 16 && lay.ncd <= 8, LMOE_ESHAPE, "lmoe_stack_decode: %d / %d chunks a thread", lay.ncg,
               lay.ncd);
  if (qtype == LMOE_Q4_0) {
    if (H == 2048)
      return small ? launch_stack<LMOE_Q4_0, 2048, 8, 4>(a, lay.lds, nb, st)
                   : launch_stack<LMOE_Q4_0, 2048, 16, 8>(a, lay.lds, nb, st);
    return small ? launch_stack<LMOE_Q4_0, 4096, 8, 4>(a, lay.lds, nb, st)
                 : launch_stack<LMOE_Q4_0, 4096, 16, 8>(a, lay.lds, nb, st);
  }
  if (H == 2048)
    return small ? launch_stack<LMOE_Q4_K, 2048, 8, 4>(a, lay.lds, nb, st)
                 : launch_stack<LMOE_Q4_K, 2048, 16, 8>(a, lay.lds, nb, st);
  return small ? launch_stack<LMOE_Q4_K, 4096, 8, 4>(a, lay.lds, nb, st)
               : launch_stack<LMOE_Q4_K, 4096, 16, 8>(a, lay.lds, nb, st);
}

// The workspace header's status word (0: every wait ended in time) read back to the host.
extern "C" int lmoe_stack_status(const void *workspace, uint32_t *status, void *stream) {
  LMOE_REQUIRE(workspace && status, LMOE_EINVAL, "lmoe_stack_status: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e = hipMemcpyAsync(status, static_cast<const uint32_t *>(workspace) + 1, 4, hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  return e == hipSuccess ? 0 : hip_fail(e, "lmoe_stack_status");
}
