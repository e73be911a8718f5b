// The decode layer's gate/up + SwiGLU and down + combine in ONE launch (lmoe_moe_fused).
//
// The three-launch chain (router GEMV, gate/up with the top-k fused in, down + combine) pays a kernel boundary
// between gate/up and down, and down then waits for its ids before its weights can be requested. Here both are
// workgroups of one grid:
//   * gate/up workgroups [0, n_gu) are k_gate_up_xr's (each wavefront ranks the token's logits, streams 2 gate + 2
//     up rows of its slot's expert, SwiGLU), and publish each wavefront's two h values as one 64-bit word
//     (f16 pair | epoch << 32) with a device-coherent store;
//   * down workgroups [n_gu, n_gu + n_dn) come after them in the grid. Each wavefront ranks the logits itself
//     (the same top-k, so the same ids and scores), requests its weight units at once (nothing in their addresses
//     depends on h), then the workgroup polls its token's h words until all carry this launch's epoch, lays them out
//     in LDS as prepared units, and finishes as k_down_xr does (the same unit dots, fma order and wavefront sum,
//     so the output is the chain's bit for bit).
// So the down weights stream while gate/up runs, and one boundary and one ids round trip leave the layer.
//
// Measured on MI355X it is the slower form, so decode keeps the two launches unless LMOE_FUSED=1: cfg2's 48-layer graph
// runs 16.2 us a layer against 14.7 (cfg5's shape 38.4 against 24.0: at H 4096 a gate/up workgroup's 83 KB of LDS
// leaves one workgroup a CU). Per-workgroup wall-clock stamps of one launch (cfg2, cold caches): gate/up workgroups
// have ranked by 2.2 us and published h by 5.5 (median) / 9.8 (last); the down workgroups see the last done word
// 0.5-1 us after it is stored and need 1.6 us more to read the h words, each a device-coherent round trip that costs
// 1.5-3 us while the weights stream, about what the kernel boundary costs. Arrival counters (one atomic a workgroup
// on 8 addresses) were slower still: their atomics completed 6-12 us after the last one was issued.
//
// Forward progress: a down workgroup waits only on gate/up workgroups, which wait on nothing and sit before it in
// the grid; workgroups are dispatched in grid order on each XCD, so every gate/up workgroup is resident or done
// by the time a down workgroup that needs it is placed. Every wait is also bounded (a wall-clock deadline): a wait
// that runs out writes NaN rows and records the launch's epoch in the status word, so a launch always ends and a
// failure is loud.
//
// Epochs without a shared counter: workgroup b keeps its own launch count in ctr[b], which no other workgroup
// touches; every launch over one workspace has the same grid, so all counts agree and ctr[b] + 1 is this launch's
// epoch in every workgroup. Words of earlier launches carry earlier epochs.
#include "lmoe_common.h"

namespace lmoe {

namespace fz {
constexpr long long kTimeoutTicks = 20000000;  // 0.2 s of the 100 MHz wall clock a wait
constexpr int kHdrWords = 64;                  // workspace header (uint32): [0] status (epoch of a timed-out launch)
constexpr int NT = 512;
constexpr int NW = NT / 64;
constexpr int RB = 2;          // rows a wavefront (gate/up: 2 gate + 2 up rows; down: 2 output rows)
constexpr int kMaxWords = 8;   // h words a down thread polls at most: ks I / 2 <= 4096 (128 units a token)

__device__ __forceinline__ uint64_t ld_word(const uint64_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_word(uint64_t *p, uint32_t payload, uint32_t ep) {
  __hip_atomic_store(p, uint64_t(payload) | (uint64_t(ep) << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_status(const uint32_t *hdr) {
  return __hip_atomic_load(hdr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void set_status(uint32_t *hdr, uint32_t ep) {
  __hip_atomic_store(hdr, ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 36 bytes at a 4-byte aligned address (a Q4_0 unit: two blocks) as 9 dwords: two 16-byte loads and one dword
typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
__device__ __forceinline__ void load_unit9(const uint8_t *p, uint32_t *u) {
  const u32x4a4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4a4 *>(p));
  const u32x4a4 b = __builtin_nontemporal_load(reinterpret_cast<const u32x4a4 *>(p + 16));
  const uint32_t c = __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(p + 32));
  u[0] = a.x, u[1] = a.y, u[2] = a.z, u[3] = a.w, u[4] = b.x, u[5] = b.y, u[6] = b.z, u[7] = b.w, u[8] = c;
}

}  // namespace fz

struct FusedArgs {
  const uint32_t *xprep;  // [T][P XS] x prepared in the gate/up type's order
  const float *logits;    // [T][ld_stride]: E routed logits (then the shared gate's when ks > k)
  int ld_stride, T, k, ks, norm;
  const uint8_t *wg, *wu, *wd;  // [E + m, I, .], [E + m, I, .], [E + m, H, .]
  int n_experts, H, I;          // routed experts E (the folded shared expert's m slices are E .. E + m - 1)
  uint32_t *ids_out;            // [T][ks]
  float *scores_out;            // [T][ks]
  uint32_t *hprep;              // [T ks][I / 64 XS] h prepared for the down type, or null (not written)
  const void *residual;
  int rdt;
  void *out;
  int odt;
  uint32_t *hdr;   // workspace: header, then ctr [n_wg], done [n_gu], then the h words
  uint32_t *ctr;
  uint32_t *done;  // [n_gu]: the epoch in which gate/up workgroup b had issued all its h words
  uint64_t *hw;    // [T ks][I / 2]
  int early;       // down workgroups request their weights before waiting for h (1) or once h is complete (0)
  int n_gu;      // gate/up workgroups (I / 8 a slot)
};

// TQ: gate/up block type (P = H / 64 units a row); TD: down block type; NPL: logits a lane (E <= 64 NPL);
// NU: h units a down lane (ks I / 64 <= 64 NU); NH: h words a down thread polls (ks I / 2 <= 256 NH).
template <int TQ, int P, int TD, int NPL, int NU, int NH>
__global__ void __launch_bounds__(fz::NT, 4) k_moe_fused(FusedArgs a) {
  using namespace fz;
  constexpr int G = 64 / P, RG = RB / G;
  constexpr int C = RB * 9 * P / 4;  // 16-byte chunks of RB rows of one gate/up matrix
  constexpr int NC = (C + 63) / 64;
  constexpr int STAGE = 2 * RB * 9 * P;  // dwords a gate/up wavefront
  constexpr int XC = 9 * P;              // 16-byte chunks of the prepared activation row
  constexpr int XPT = (XC + NT - 1) / NT;
  constexpr int HH = TD == LMOE_Q4_K ? 32 : 16;  // h's prepared order (the down type's nibble words)
  // LDS: gate/up: the activation row and NW stages; down: the token's h units (32 pair dwords each, <= 128 units);
  // both: NW x 64 dwords of top-k scratch
  constexpr int GU_DW = XC * 4 + NW * STAGE, DN_DW = 128 * 32;
  __shared__ u32x4 lds4[(GU_DW > DN_DW ? GU_DW : DN_DW) / 4];
  __shared__ __attribute__((aligned(16))) uint32_t scr_all[NW][64];
  __shared__ uint32_t ep_lds;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int b = blockIdx.x;
  uint32_t *scr = scr_all[wave];
  // this launch's epoch: one more than this workgroup's own count of launches (see the file comment). Thread 0
  // reads the count, stores the new one and hands the epoch to the other threads through LDS at the workgroup's
  // first barrier (a thread that read ctr[b] itself could see thread 0's new count)
  const uint32_t count = a.ctr[b];
  const int m = a.ks - a.k;            // folded shared-expert slices a token
  const int ne = a.n_experts + m;      // experts the weight buffers hold
  const int I = a.I, H = a.H;

  if (b < a.n_gu) {
    // ---- gate/up + SwiGLU: k_gate_up_xr<TQ, P, RB, NPL> ------------------------------------------------------
    const int gx = I / (NW * RB);
    const int s = b / gx, bx = b - s * gx;
    const int r0 = (bx * NW + wave) * RB;
    const int g = lane / P, p = lane % P;
    u32x4 *xl = lds4;
    uint32_t *stage = reinterpret_cast<uint32_t *>(lds4 + XC) + wave * STAGE;
    const size_t xrow = size_t(s / a.ks);
    const int jslot = s % a.ks;
    const bool shared_slot = jslot >= a.k;  // uniform across the workgroup
    const float *row = a.logits + xrow * a.ld_stride;
    float v[NPL];
#pragma unroll
    for (int j = 0; j < NPL; ++j) v[j] = row[min(lane + 64 * j, a.n_experts - 1)];
    const u32x4 *xg4 = reinterpret_cast<const u32x4 *>(a.xprep + xrow * P * XS);
    u32x4 xc[XPT];
#pragma unroll
    for (int i = 0; i < XPT; ++i) xc[i] = xg4[min(int(threadIdx.x) + NT * i, XC - 1)];
    uint32_t e;
    if (shared_slot) {
      e = uint32_t(a.n_experts + jslot - a.k);
      if (bx == 0 && wave == 0 && lane == 0) {
        a.ids_out[s] = e;
        a.scores_out[s] = sigmoidf_(row[a.n_experts]);
      }
    } else {
      uint32_t id;
      if (bx == 0 && wave == 0) {
        float sc;
        topk_wave<NPL, true>(v, a.n_experts, a.k, a.norm, scr, &id, &sc);
        if (lane == jslot) {
          a.ids_out[s] = id;
          a.scores_out[s] = sc;
        }
        id = uint32_t(__builtin_amdgcn_readlane(int(id), jslot));
      } else {
        topk_wave<NPL, false>(v, a.n_experts, a.k, a.norm, scr, &id, nullptr, jslot);
      }
      e = id;
    }
    const bool valid = e < uint32_t(a.n_experts) || shared_slot;
    const size_t rsafe = size_t(valid ? e : 0u) * I + r0;
    const u32x4 *gsrc = reinterpret_cast<const u32x4 *>(a.wg + rsafe * (36 * P));
    const u32x4 *usrc = reinterpret_cast<const u32x4 *>(a.wu + rsafe * (36 * P));
    u32x4 vg[NC], vu[NC];
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = min(lane + 64 * i, C - 1);
      vg[i] = __builtin_nontemporal_load(gsrc + c);
      vu[i] = __builtin_nontemporal_load(usrc + c);
    }
#pragma unroll
    for (int i = 0; i < XPT; ++i) xl[min(int(threadIdx.x) + NT * i, XC - 1)] = xc[i];
    if (threadIdx.x == 0) {
      ep_lds = count + 1u;
      a.ctr[b] = count + 1u;
    }
    __syncthreads();
    const uint32_t ep = ep_lds;
    u32x4 *st4 = reinterpret_cast<u32x4 *>(stage);
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = min(lane + 64 * i, C - 1);
      st4[c] = vg[i];
      st4[C + c] = vu[i];
    }
    __builtin_amdgcn_wave_barrier();
    float hv[RG];
    if (!valid) {
#pragma unroll
      for (int i = 0; i < RG; ++i) hv[i] = 0.0f;
    } else {
      uint32_t xv[32];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const u32x4 q = xl[9 * p + i];
        xv[4 * i] = q.x;
        xv[4 * i + 1] = q.y;
        xv[4 * i + 2] = q.z;
        xv[4 * i + 3] = q.w;
      }
      const u32x4 qs = xl[9 * p + 8];
      const float sx0 = __uint_as_float(qs.x), sx1 = __uint_as_float(qs.y);
      float pg[RG], pu[RG];
#pragma unroll
      for (int i = 0; i < RG; ++i) {
        const int rr = g + G * i;
        pg[i] = row_unit_dot_r<TQ>(stage + rr * 9 * P, p, xv, sx0, sx1);
        pu[i] = row_unit_dot_r<TQ>(stage + (RB + rr) * 9 * P, p, xv, sx0, sx1);
      }
#pragma unroll
      for (int i = 0; i < RG; ++i) hv[i] = silu_mul(group_sum<P>(pg[i]), group_sum<P>(pu[i]));
    }
    // rows r0 (group 0, i = 0) and r0 + 1 (P = 32: group 1; P = 64: i = 1) as one f16 pair word
    // each rounded to fp32 first, then to f16, as the chain stores it
    const float h0 = opaque(hv[0]);
    const float h1 = opaque(RG == 2 ? hv[RG - 1] : __shfl(hv[0], 32, 64));
    if (lane == 0) {
      const _Float16 f0 = _Float16(h0), f1 = _Float16(h1);
      const uint32_t pr = uint32_t(__builtin_bit_cast(uint16_t, f0)) | (uint32_t(__builtin_bit_cast(uint16_t, f1)) << 16);
      st_word(a.hw + size_t(s) * (I / 2) + r0 / 2, pr, ep);
      if (a.hprep) {
        _Float16 *hp = reinterpret_cast<_Float16 *>(a.hprep + (size_t(s) * (I / 64) + (r0 >> 6)) * XS);
        int dw, half;
        xslot(r0 & 63, HH, &dw, &half);
        hp[2 * dw + half] = f0;
        xslot((r0 + 1) & 63, HH, &dw, &half);
        hp[2 * dw + half] = f1;
      }
    }
    // the workgroup's done word, stored once its wavefronts have issued their h words: it tells the down workgroups
    // when to read them, the words' own epochs decide what they read (relaxed stores carry no order)
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_store(a.done + b, ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }

  // ---- down + weighted combine + residual: k_down_xr<TD, NU, ., 1> with h polled ------------------------------
  const int d = b - a.n_gu;
  const int nrb = H / (NW * RB);
  const int t = d / nrb, bx = d - t * nrb;
  const int n0 = (bx * NW + wave) * RB;
  const int PI = I / 64, U = a.ks * PI;
  const float *row = a.logits + size_t(t) * a.ld_stride;
  float v[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) v[j] = row[min(lane + 64 * j, a.n_experts - 1)];
  const float gate_logit = m > 0 ? row[a.n_experts] : 0.0f;
  // 1. the token's picks, ranked by this wavefront (the gate/up workgroups' top-k: the same ids and scores);
  // lane j < ks then holds slot j's expert and weight
  uint32_t my_id;
  float my_sc;
  topk_wave<NPL, true>(v, a.n_experts, a.k, a.norm, scr, &my_id, &my_sc);
  if (lane >= a.k) {
    my_id = uint32_t(a.n_experts + lane - a.k);
    my_sc = sigmoidf_(gate_logit);
  }
  // 2. this lane's units (slot ja, unit pa) and their weights at rows n0, n0 + 1, straight into registers: at once
  // (early) or after h is complete
  int ja[NU], pa[NU];
  float fa[NU];
  uint32_t es[NU];
  constexpr int WD = TD == LMOE_Q4_K ? 12 : 9;  // dwords a unit a row in registers (Q4_K: header + pair's qs)
  uint32_t w[NU][RB][WD];
  const size_t rowb = size_t(36) * PI;
#pragma unroll
  for (int q = 0; q < NU; ++q) {
    const int u = lane + 64 * q, uc = min(u, U - 1);
    ja[q] = uc / PI;
    pa[q] = uc - ja[q] * PI;
    const uint32_t e = uint32_t(__shfl(int(my_id), ja[q], 64));
    const float sj = __shfl(my_sc, ja[q], 64);
    fa[q] = (u < U && e < uint32_t(ne)) ? sj : 0.0f;
    es[q] = e < uint32_t(ne) ? e : 0u;
  }
  auto load_w = [&]() {
#pragma unroll
    for (int q = 0; q < NU; ++q) {
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const uint8_t *rp = a.wd + (size_t(es[q]) * H + n0 + r) * rowb;
        if (TD == LMOE_Q4_0) {
          load_unit9(rp + 36 * pa[q], w[q][r]);
        } else {
          const u32x4 *sb = reinterpret_cast<const u32x4 *>(rp + 144 * (pa[q] >> 2));
          const u32x4 h4 = __builtin_nontemporal_load(sb);
          const u32x4 q0 = __builtin_nontemporal_load(sb + 1 + 2 * (pa[q] & 3));
          const u32x4 q1 = __builtin_nontemporal_load(sb + 2 + 2 * (pa[q] & 3));
          w[q][r][0] = h4.x, w[q][r][1] = h4.y, w[q][r][2] = h4.z, w[q][r][3] = h4.w;
          w[q][r][4] = q0.x, w[q][r][5] = q0.y, w[q][r][6] = q0.z, w[q][r][7] = q0.w;
          w[q][r][8] = q1.x, w[q][r][9] = q1.y, w[q][r][10] = q1.z, w[q][r][11] = q1.w;
        }
      }
    }
  };
  if (a.early) load_w();
  asm volatile("" ::: "memory");
  if (threadIdx.x == 0) {
    ep_lds = count + 1u;
    a.ctr[b] = count + 1u;
  }
  __syncthreads();
  const uint32_t ep = ep_lds;
  // 3. the done words of the token's gate/up workgroups (one a thread), polled until each carries this epoch
  bool ok = true;
  {
    const int gpt = a.ks * (I / (NW * RB));  // the token's gate/up workgroups: [t gpt, (t + 1) gpt)
    const uint32_t *dp = a.done + size_t(t) * gpt;
    for (int i0 = 0; i0 < gpt && ok; i0 += NT) {
      const int i = min(i0 + int(threadIdx.x), gpt - 1);
      const long long t0 = wall_clock64();
      for (int it = 0;; ++it) {
        if (__hip_atomic_load(dp + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == ep) break;
        __builtin_amdgcn_s_sleep(1);
        if ((it & 15) == 15) {
          if (ld_status(a.hdr) == ep) {  // another workgroup's wait ran out in this launch
            ok = false;
            break;
          }
          if (wall_clock64() - t0 > kTimeoutTicks) {
            set_status(a.hdr, ep);
            ok = false;
            break;
          }
        }
      }
    }
  }
  if (__syncthreads_or(!ok)) {  // a wait ran out: NaN rows, the launch's epoch already in the status word
    if (lane < RB) store_elt(a.out, size_t(t) * H + n0 + lane, __builtin_nanf(""), a.odt);
    return;
  }
  if (!a.early) load_w();
  // 4. the token's h words, read until every one carries this launch's epoch (all do by now, but for a word whose
  // store is still on its way), into LDS as prepared pair units
  const int nwd = a.ks * (I / 2);
  const uint64_t *src = a.hw + size_t(t) * nwd;
  uint64_t hwv[NH];
#pragma unroll
  for (int q = 0; q < NH; ++q) hwv[q] = ld_word(src + min(int(threadIdx.x) + NT * q, nwd - 1));
  {
    const long long t0 = wall_clock64();
    for (int it = 0;; ++it) {
      uint32_t pend = 0;
#pragma unroll
      for (int q = 0; q < NH; ++q)
        if (int(threadIdx.x) + NT * q < nwd && uint32_t(hwv[q] >> 32) != ep) pend |= 1u << q;
      if (!pend) break;
      __builtin_amdgcn_s_sleep(1);
      if ((it & 15) == 15) {
        if (ld_status(a.hdr) == ep) {  // another workgroup's wait ran out in this launch
          ok = false;
          break;
        }
        if (wall_clock64() - t0 > kTimeoutTicks) {
          set_status(a.hdr, ep);
          ok = false;
          break;
        }
      }
#pragma unroll
      for (int q = 0; q < NH; ++q)
        if ((pend >> q) & 1u) hwv[q] = ld_word(src + threadIdx.x + NT * q);
    }
  }
  // word i (rows 2 i', 2 i' + 1 of slot i / (I / 2), i' = i mod I / 2) lands in LDS unit i / 32 (units are laid out
  // slot-major, I / 64 a slot, like the words), at the pair slots of rows 2 (i mod 32) and + 1 of that unit; i mod 32
  // is this thread's lane mod 32 for every word it holds
  uint16_t *hl = reinterpret_cast<uint16_t *>(lds4);
  int dw0, hf0, dw1, hf1;
  xslot(2 * (lane & 31), HH, &dw0, &hf0);
  xslot(2 * (lane & 31) + 1, HH, &dw1, &hf1);
  const int o0 = 2 * dw0 + hf0, o1 = 2 * dw1 + hf1;
#pragma unroll
  for (int q = 0; q < NH; ++q) {
    const int i = int(threadIdx.x) + NT * q;
    if (i < nwd) {
      uint16_t *u = hl + (i >> 5) * 64;
      u[o0] = uint16_t(hwv[q]);
      u[o1] = uint16_t(hwv[q] >> 16);
    }
  }
  if (__syncthreads_or(!ok)) {  // a wait ran out: NaN rows, the launch's epoch already in the status word
    if (lane < RB) store_elt(a.out, size_t(t) * H + n0 + lane, __builtin_nanf(""), a.odt);
    return;
  }
  // 5. each unit's pairs and half sums (k_down_xr's step 3)
  const h2_t one2 = {_Float16(1.0f), _Float16(1.0f)};
  const u32x4 *hl4 = reinterpret_cast<const u32x4 *>(lds4);
  float acc[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) acc[r] = 0.0f;
#pragma unroll
  for (int q = 0; q < NU; ++q) {
    // one unit's pairs live at a time (the weights of every unit are already in registers)
    if (q > 0) __builtin_amdgcn_sched_barrier(0);
    const int uc = ja[q] * PI + pa[q];
    uint32_t xv[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const u32x4 h4 = hl4[uc * 8 + i];
      xv[4 * i] = h4.x, xv[4 * i + 1] = h4.y, xv[4 * i + 2] = h4.z, xv[4 * i + 3] = h4.w;
    }
    float x0 = 0.0f, x1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t d0 = TD == LMOE_Q4_K ? xv[2 * i] : xv[i];
      const uint32_t d1 = TD == LMOE_Q4_K ? xv[2 * i + 1] : xv[16 + i];
      x0 = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, d0), one2, x0, false);
      x1 = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, d1), one2, x1, false);
    }
    // 6. dots, in k_down_xr's order (unit-major, rows inner)
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      float dv;
      if (TD == LMOE_Q4_0)
        dv = unit_dot_q4_0(w[q][r], xv, x0, x1);
      else
        dv = unit_dot_q4_k(w[q][r], w[q][r] + 4, pa[q] & 3, xv, x0, x1);
      acc[r] = fmaf(fa[q], dv, acc[r]);
    }
  }
  // 7. the rows' sums, residual, out
#pragma unroll
  for (int r = 0; r < RB; ++r) acc[r] = wave_sum(acc[r]);
  if (lane < RB) {
    float vo = acc[0];
#pragma unroll
    for (int r = 1; r < RB; ++r) vo = lane == r ? acc[r] : vo;
    const size_t o = size_t(t) * H + n0 + lane;
    if (a.residual) vo += load_elt(a.residual, o, a.rdt);
    store_elt(a.out, o, vo, a.odt);
  }
}

namespace {

int fused_grid(int T, int ks, int H, int I, int *n_gu) {
  *n_gu = T * ks * (I / (fz::NW * fz::RB));
  return *n_gu + T * (H / (fz::NW * fz::RB));
}

size_t fused_ctr_words(int n_wg) { return (size_t(n_wg) + 63) / 64 * 64; }

// Whether the down workgroups request their weights before h is complete (the default) or once it is
// (LMOE_FUSED_EARLY=0). cfg2's 48-layer graph: 16.2 against 20.5 us a layer; the early requests do lengthen gate/up's
// tail (its last h word 7.2 -> 9.8 us after the launch) but take the weight latency off the path after the hand-off.
bool fused_early() {
  static const bool v = [] {
    const char *e = getenv("LMOE_FUSED_EARLY");
    return !(e && e[0] == '0');
  }();
  return v;
}

}  // namespace

}  // namespace lmoe

using namespace lmoe;

extern "C" size_t lmoe_moe_fused_workspace_bytes(int T, int k, int n_shared, int H, int I) {
  if (T <= 0 || k <= 0 || n_shared < 0 || H <= 0 || I <= 0) return 0;
  int n_gu = 0;
  const int n_wg = fused_grid(T, k + n_shared, H, I, &n_gu);
  return 4 * (size_t(fz::kHdrWords) + 2 * fused_ctr_words(n_wg)) + 8 * size_t(T) * (k + n_shared) * (I / 2);
}

extern "C" int lmoe_moe_fused(const float *logits, int ld_stride, int T, int k, int norm, const uint32_t *x_prep,
                              const uint8_t *wg, const uint8_t *wu, const uint8_t *wd, int tq, int td, int n_experts,
                              int H, int I, int n_shared, uint32_t *ids_out, float *scores_out, uint32_t *hprep,
                              const void *residual, int rdtype, void *out, int odtype, void *workspace,
                              size_t workspace_bytes, void *stream) {
  static const char *fn = "lmoe_moe_fused";
  LMOE_REQUIRE(qtype_ok(tq) && td == tq, LMOE_ETYPE, "%s: ggml types %d/%d (all three Q4_0 = 2, or all Q4_K = 12)",
               fn, tq, td);
  LMOE_REQUIRE(H == 2048 || H == 4096, LMOE_ESHAPE, "%s: hidden %d (2048 or 4096)", fn, H);
  LMOE_REQUIRE(T >= 1 && T <= 16 && k >= 1 && k <= 32 && n_shared >= 0 && k + n_shared <= 64 && k <= n_experts &&
                   n_experts <= 1024,
               LMOE_ESHAPE, "%s: %d tokens, top-%d of %d experts and %d shared slices", fn, T, k, n_experts,
               n_shared);
  LMOE_REQUIRE(I % 64 == 0 && (td != LMOE_Q4_K || I % 256 == 0) && I % (fz::NW * fz::RB) == 0, LMOE_ESHAPE,
               "%s: width %d", fn, I);
  const int ks = k + n_shared, PI = I / 64;
  LMOE_REQUIRE(ks * PI <= 128 && size_t(ks) * (I / 2) <= size_t(fz::NT) * fz::kMaxWords, LMOE_ESHAPE,
               "%s: %d h units a token (at most 128)", fn, ks * PI);
  LMOE_REQUIRE(dtype_ok(odtype) && (!residual || dtype_ok(rdtype)), LMOE_EINVAL, "%s: bad dtype", fn);
  LMOE_REQUIRE(logits && x_prep && wg && wu && wd && ids_out && scores_out && out && workspace, LMOE_EINVAL,
               "%s: null pointer", fn);
  LMOE_REQUIRE(aligned16(wg) && aligned16(wu) && aligned16(wd) && aligned16(x_prep) && aligned16(workspace) &&
                   (!hprep || aligned16(hprep)),
               LMOE_EALIGN, "%s: buffers must be 16-byte aligned", fn);
  LMOE_REQUIRE(ld_stride >= n_experts + (n_shared > 0 ? 1 : 0), LMOE_ESHAPE, "%s: logits stride %d", fn, ld_stride);
  LMOE_REQUIRE(workspace_bytes >= lmoe_moe_fused_workspace_bytes(T, k, n_shared, H, I), LMOE_ESHAPE,
               "%s: workspace of %zu bytes (needs %zu)", fn, workspace_bytes,
               lmoe_moe_fused_workspace_bytes(T, k, n_shared, H, I));
  FusedArgs a{};
  a.xprep = x_prep, a.logits = logits, a.ld_stride = ld_stride, a.T = T, a.k = k, a.ks = ks, a.norm = norm;
  a.wg = wg, a.wu = wu, a.wd = wd, a.n_experts = n_experts, a.H = H, a.I = I;
  a.ids_out = ids_out, a.scores_out = scores_out, a.hprep = hprep;
  a.residual = residual, a.rdt = rdtype, a.out = out, a.odt = odtype;
  int n_gu = 0;
  const int n_wg = fused_grid(T, ks, H, I, &n_gu);
  a.n_gu = n_gu;
  a.hdr = static_cast<uint32_t *>(workspace);
  a.ctr = a.hdr + fz::kHdrWords;
  a.done = a.ctr + fused_ctr_words(n_wg);
  a.hw = reinterpret_cast<uint64_t *>(a.done + fused_ctr_words(n_wg));
  a.early = fused_early();
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int NU = ks * PI <= 64 ? 1 : 2;
  const int nh = (ks * (I / 2) + fz::NT - 1) / fz::NT;
  auto go = [&](auto tqc, auto pc, auto tdc, auto nplc, auto nuc) {
    constexpr int TQ = decltype(tqc)::value, P = decltype(pc)::value, TD = decltype(tdc)::value;
    constexpr int NPL = decltype(nplc)::value, N = decltype(nuc)::value;
    if (nh <= 4)
      launch(k_moe_fused<TQ, P, TD, NPL, N, 4>, dim3(n_wg), dim3(fz::NT), 0, st, a);
    else
      launch(k_moe_fused<TQ, P, TD, NPL, N, 8>, dim3(n_wg), dim3(fz::NT), 0, st, a);
  };
  using Q0 = std::integral_constant<int, LMOE_Q4_0>;
  using QK = std::integral_constant<int, LMOE_Q4_K>;
  auto by_nu = [&](auto tqc, auto pc, auto tdc, auto nplc) {
    if (NU == 1) go(tqc, pc, tdc, nplc, std::integral_constant<int, 1>());
    else go(tqc, pc, tdc, nplc, std::integral_constant<int, 2>());
  };
  auto by_npl = [&](auto tqc, auto pc, auto tdc) {
    if (n_experts <= 64) by_nu(tqc, pc, tdc, std::integral_constant<int, 1>());
    else if (n_experts <= 128) by_nu(tqc, pc, tdc, std::integral_constant<int, 2>());
    else if (n_experts <= 256) by_nu(tqc, pc, tdc, std::integral_constant<int, 4>());
    else if (n_experts <= 512) by_nu(tqc, pc, tdc, std::integral_constant<int, 8>());
    else by_nu(tqc, pc, tdc, std::integral_constant<int, 16>());
  };
  auto by_td = [&](auto tqc, auto pc) { by_npl(tqc, pc, tqc); };
  auto by_p = [&](auto tqc) {
    if (H == 2048) by_td(tqc, std::integral_constant<int, 32>());
    else by_td(tqc, std::integral_constant<int, 64>());
  };
  if (tq == LMOE_Q4_0) by_p(Q0());
  else by_p(QK());
  LMOE_LAUNCHED(fn);
  return 0;
}

// The status word of a fused decode workspace: 0, or the epoch of the last launch whose h wait ran out (its output
// rows are NaN). Synchronises the stream.
extern "C" int lmoe_moe_fused_status(const void *workspace, uint32_t *status, void *stream) {
  LMOE_REQUIRE(workspace && status, LMOE_EINVAL, "lmoe_moe_fused_status: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e = hipMemcpyAsync(status, workspace, 4, hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  return e == hipSuccess ? 0 : hip_fail(e, "lmoe_moe_fused_status");
}
