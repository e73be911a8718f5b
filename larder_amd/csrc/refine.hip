// The prefill router's picks made exact: the router GEMM's logits narrowed to a candidate set with a proven error
// bound, the candidates' logits recomputed in the decode router's fixed order, the top-k taken on those.
//
// The prefill router logits come from an MFMA GEMM on f16 operands (k_router_gemm): fast, but its summation order is
// the matrix core's, which nothing restates. The decode router (k_router_gemv) sums in a fixed order that the test
// oracle restates bit for bit: thread t of 256 forms the fma chain of its 8-element items t, t + 256, ... of x . w
// from zero, each wavefront adds its 64 chains as a balanced tree (wave_sum), and the four wavefront totals are added
// left to right. Here, for each token:
//   * M_j (the GEMM's logit) and L_j (the fixed-order logit) of expert j differ by at most
//       e_j = (g A + C + D) a_j + A d_j + B c_j + c B b_j
//     with, per token, A = |f16(x)|, B = |x|, C = |f16(x) - x|, D = |f16(x) restricted to f16 subnormals| and, per
//     router row, a = |f16(w)|, b = |w|, c = |f16(w) - w|, d = |f16(w) restricted to f16 subnormals| (2-norms, which
//     bound the sums of |x_i w_i| by Cauchy-Schwarz), g = (H / ks + ks + 64) 2^-23 (M is the sum from zero, in slice
//     order, of ks slices of H / ks exact f16 products each, every slice summed by the matrix core in some order:
//     any summation tree over n terms is at most n - 1 additions deep, so each product meets at most
//     H / ks + ks - 2 additions on its way to M, each off by at most 2 units of fp32 rounding; 64 more for the
//     second-order terms) and c = 48 2^-24 (the fixed order's additions: at most 32 chain steps, a 6-level tree and
//     3 more adds).
//     The D and d terms cover a matrix core that flushes f16 subnormal inputs; C and c the f16 rounding of bf16 / f32
//     inputs. e_j is taken 1 % larger, plus two fp32 units of |M_j|, so that its own rounding cannot shrink it;
//   * tau = the k-th largest of M_j - e_j; every expert with M_j + e_j >= tau is a candidate. Any expert outside that
//     set has L_j <= M_j + e_j < tau <= the k-th largest L, so the top-k of L (ties to the lower index) lies inside
//     the candidate set, and every expert tied with the k-th L is in it too;
//   * a candidate whose interval [M_j - e_j, M_j + e_j] meets another candidate's gets L_j recomputed in the fixed
//     order (one wavefront a token standing in for the four wavefronts of k_router_gemv: lane l forms the chains of
//     threads l, l + 64, l + 128, l + 192); two disjoint intervals already order their experts as L would. The top-k
//     is taken over v_j = L_j (recomputed) or M_j (the rest): the ids are exactly the top-k of L, i.e. of the decode
//     router on the same x. With a NaN logit, a token whose bound is not finite (|x| past f16), or more than 64
//     candidates, every expert is recomputed.
// The token's norms are summed in fp32 (off by at most ~1e-6 relative, far inside the 1 % margin); the rows' norms
// once a layer in fp64. The shared expert's gate row (when given) is recomputed in the fixed order for every token. Scores are the softmax
// terms of v (renormalised over the picks when norm): those of the picks are exact fixed-order logits; the
// denominator without renormalisation also holds the other experts' GEMM logits.
#include "lmoe_common.h"

namespace lmoe {

namespace rf {
constexpr int NT = 256;
constexpr int kMaxH = 8192;
constexpr int kMaxE = 1024;
}  // namespace rf

// Row norms of the router weight as the two routers see it: out[r] = {|f16(w_r)|, |w_r|, |f16(w_r) - w_r|,
// |f16(w_r) restricted to f16 subnormals|}, rounded up to float. Rows E (and E + 1 with the shared gate row wsg). One
// workgroup a row, fp64 sums.
__global__ void __launch_bounds__(256) k_router_norms(const void *wr, const void *wsg, int wdt, int E, int H,
                                                      float *out) {
  __shared__ double red[4][4];
  const int r = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const void *row = r < E ? static_cast<const char *>(wr) + size_t(r) * H * (wdt == LMOE_F32 ? 4 : 2) : wsg;
  double s[4] = {0.0, 0.0, 0.0, 0.0};
  for (int i = threadIdx.x; i < H; i += 256) {
    const float w = load_elt(row, size_t(i), wdt);
    const float wh = float(_Float16(w));
    const double d = double(wh) - double(w);
    s[0] += double(wh) * wh;
    s[1] += double(w) * w;
    s[2] += d * d;
    if (wh != 0.0f && fabsf(wh) < 6.103515625e-05f) s[3] += double(wh) * wh;
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    for (int o = 32; o > 0; o >>= 1) s[q] += __shfl_xor(s[q], o, 64);
    if (lane == 0) red[wave][q] = s[q];
  }
  __syncthreads();
  if (threadIdx.x < 4) {
    const int q = threadIdx.x;
    const double t = (red[0][q] + red[1][q]) + (red[2][q] + red[3][q]);
    const float f = float(sqrt(t));
    // rounded up: the next float above (the sum's own error is far below one fp32 unit)
    out[size_t(r) * 4 + q] = f > 0.0f && isfinite(f) ? __uint_as_float(__float_as_uint(f) + 1u) : f;
  }
}

struct RefineArgs {
  const float *part;  // ks slices [ks][T][ldp] of the router GEMM, or the logits [T][ldp] when ks == 1
  int ks, ldp;
  const void *x;  // [T][H] raw, xdt
  int xdt, T, H;
  const void *wr, *wsg;  // [E][H], [H] (or null), wdt
  int wdt, E;
  const float *norms;  // [E (+1)][4] (k_router_norms)
  int k, norm, m;      // top-k, renormalise, folded shared slices
  uint32_t *ids;       // [T][k + m]
  float *scores;       // [T][k + m]
  float *logits;       // [T][E]: v (candidates' fixed-order logits, the GEMM's elsewhere), or null
  float *gate;         // [T]: the shared gate's fixed-order logit, or null
  int *n_cand;         // [T]: candidates, or null
};

// One token a wavefront, four a workgroup, no barriers (each wavefront's LDS is its own). KS: the K slices of the
// router GEMM (1: its logits); XC: 8-element items of a row each of k_router_gemv's threads holds (H / 8 / 256
// rounded up, at most 4). Lane l stands in for that kernel's threads l, l + 64, l + 128, l + 192 (its four
// wavefronts' lane l): it loads their x items l + 64 q + 256 i (which cover x once, for the norms) into the
// wavefront's LDS and forms their four chains for every recomputed row.
template <int NPL, int WDT, int KS, int XC>
__global__ void __launch_bounds__(rf::NT) k_router_refine(RefineArgs a) {
  using namespace rf;
  constexpr int WQ = WDT == LMOE_F32 ? 2 : 1;  // 16-byte pieces of an 8-weight item
  constexpr int TB = XC * WQ >= 4 ? 1 : 2;     // fixed-order rows a batch (<= 16 loads in flight a lane)
  constexpr int NCW = 64;                      // candidates a wavefront ranks itself (more: all recomputed)
  // dynamic LDS: [4][E] v by expert (the fixed-order logit where recomputed, else M), then [4][H] each wavefront's
  // token's x as stored (xdt)
  extern __shared__ __attribute__((aligned(16))) float dyn[];
  __shared__ uint16_t cidx[4][NCW];
  __shared__ float clo[4][NCW], chi[4][NCW];
  __shared__ uint32_t ckey[4][NCW];
  __shared__ uint16_t ridx[4][NCW + 1];
  __shared__ __attribute__((aligned(16))) uint32_t scr[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + wave;
  if (t >= a.T) return;
  const int E = a.E, H = a.H, nit = H / 8;
  const int wsz = WDT == LMOE_F32 ? 4 : 2;
  const int xsz = a.xdt == LMOE_F32 ? 4 : 2;
  const int ev = (E + 3) & ~3;
  float *vf = dyn + wave * ev;
  u32x4 *xl4 = reinterpret_cast<u32x4 *>(dyn + 4 * ev) + size_t(wave) * (H * xsz / 16);
  // 1. every load first: the GEMM's slices, the rows' norms, this lane's x items
  float p[KS][NPL];
#pragma unroll
  for (int q = 0; q < KS; ++q) {
    const float *prow = a.part + (size_t(q) * a.T + t) * a.ldp;
#pragma unroll
    for (int j = 0; j < NPL; ++j) p[q][j] = prow[min(lane + 64 * j, E - 1)];
  }
  const int xq = a.xdt == LMOE_F32 ? 2 : 1;
  const u32x4 *x4 = reinterpret_cast<const u32x4 *>(static_cast<const char *>(a.x) + size_t(t) * H * (2 * xq));
  u32x4 xc[4][XC][2];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int i = 0; i < XC; ++i) {
      const int it = min(lane + 64 * q + 256 * i, nit - 1);
      xc[q][i][0] = x4[it * xq];
      xc[q][i][1] = x4[it * xq + xq - 1];
    }
  float4 nw[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) nw[j] = reinterpret_cast<const float4 *>(a.norms)[min(lane + 64 * j, E - 1)];
  // M: the slices added in slice order from zero (k_router_finish's sums)
  float mv[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < KS; ++q) s += p[q][j];
    mv[j] = s;
    if (lane + 64 * j < E) vf[lane + 64 * j] = s;
  }
  // 2. x into the wavefront's LDS as stored, and the token's squared norms in fp32 (at most ~1e-6 relative off: far
  // inside the bound's 1 % margin)
  float s4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int i = 0; i < XC; ++i) {
      const int it = lane + 64 * q + 256 * i;
      if (it < nit) {
        float xv[8];
        unpack8(xc[q][i][0], xc[q][i][1], a.xdt, xv);
        xl4[it * xq] = xc[q][i][0];
        xl4[it * xq + xq - 1] = xc[q][i][1];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float xh = float(_Float16(xv[e])), d = xh - xv[e];
          s4[0] = fmaf(xh, xh, s4[0]);
          s4[1] = fmaf(xv[e], xv[e], s4[1]);
          s4[2] = fmaf(d, d, s4[2]);
          s4[3] = (xh != 0.0f && fabsf(xh) < 6.103515625e-05f) ? fmaf(xh, xh, s4[3]) : s4[3];
        }
      }
    }
  float nrm[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) nrm[q] = sqrtf(wave_sum(s4[q])) * 1.0001f;
  // 3. the bound, tau, the candidates, and among them the ones to recompute: those whose interval [M - e, M + e] meets
  // another candidate's (two disjoint intervals order their experts as the exact logits would)
  const float A = nrm[0], B = nrm[1], C = nrm[2], D = nrm[3];
  const float g = float(H / KS + KS + 64) * 1.1920928955078125e-07f, cg = 48.0f * 5.9604644775390625e-08f;
  const float s1 = g * A + C + D, s2 = cg * B;
  float lo[NPL], hi[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    float eb = s1 * nw[j].x + A * nw[j].w + B * nw[j].z + s2 * nw[j].y;
    eb = eb * 1.01f + 2.384185791015625e-07f * fabsf(mv[j]);
    const bool wide = !isfinite(eb) || mv[j] != mv[j];
    lo[j] = wide ? -INFINITY : mv[j] - eb;
    hi[j] = wide ? INFINITY : mv[j] + eb;
  }
  const uint32_t kid = rank_pick_wave<NPL>(lo, E, a.k - 1);  // the expert holding the k-th lo
  float tau = -INFINITY;
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const float lk = __shfl(lo[j], int(kid & 63u), 64);
    if (kid < uint32_t(E) && int(kid >> 6) == j) tau = lk;
  }
  int n = 0;
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const bool in = lane + 64 * j < E && hi[j] >= tau;
    const uint64_t bal = __ballot(in);
    const int at = n + __popcll(bal & ((uint64_t(1) << lane) - 1));
    if (in && at < NCW) {
      cidx[wave][at] = uint16_t(lane + 64 * j);
      clo[wave][at] = lo[j];
      chi[wave][at] = hi[j];
    }
    n += __popcll(bal);
  }
  __builtin_amdgcn_wave_barrier();
  const bool all = n > NCW;  // every expert recomputed (the top-k of v then over all of them)
  int nr = 0;
  if (!all) {
    bool rec = false;
    if (lane < n) {
      const float l = clo[wave][lane], h = chi[wave][lane];
      for (int o = 0; o < n; ++o) rec |= o != lane && clo[wave][o] <= h && l <= chi[wave][o];
    }
    const uint64_t bal = __ballot(rec);
    if (rec) ridx[wave][__popcll(bal & ((uint64_t(1) << lane) - 1))] = cidx[wave][lane];
    nr = __popcll(bal);
  }
  const int rows = all ? E : nr;               // rows 0 .. rows - 1 (by expert when all)
  const int tasks = rows + (a.wsg ? 1 : 0);    // the shared gate row last
  __builtin_amdgcn_wave_barrier();
  // 4. the recomputed rows' fixed-order logits, TB rows a batch with all their loads out first; lane l's chains are
  // k_router_gemv's threads l + 64 q, the wavefront tree over each q, then the four totals left to right
  float gl = 0.0f;
  for (int b0 = 0; b0 < tasks; b0 += TB) {
    u32x4 wq[TB][4][XC][WQ];
    int er[TB];
#pragma unroll
    for (int r = 0; r < TB; ++r) {
      const int task = min(b0 + r, tasks - 1);
      er[r] = task >= rows ? E : (all ? task : int(ridx[wave][task]));
      const u32x4 *w4 = reinterpret_cast<const u32x4 *>(
          er[r] < E ? static_cast<const char *>(a.wr) + size_t(er[r]) * H * wsz : static_cast<const char *>(a.wsg));
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int i = 0; i < XC; ++i) {
          const int it = min(lane + 64 * q + 256 * i, nit - 1);
#pragma unroll
          for (int h = 0; h < WQ; ++h) wq[r][q][i][h] = __builtin_nontemporal_load(w4 + it * WQ + h);
        }
    }
#pragma unroll
    for (int r = 0; r < TB; ++r) {
      float part[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < XC; ++i) {
          const int it = lane + 64 * q + 256 * i;
          if (it < nit) {  // a thread past the row's items adds nothing
            float wv[8], xv[8];
            unpack8(wq[r][q][i][0], wq[r][q][i][WQ - 1], WDT, wv);
            unpack8(xl4[it * xq], xl4[it * xq + xq - 1], a.xdt, xv);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc = fmaf(xv[e], wv[e], acc);
          }
        }
        part[q] = wave_sum(acc);
      }
      const float l = ((part[0] + part[1]) + part[2]) + part[3];
      if (b0 + r < tasks) {
        if (er[r] < E) {
          if (lane == 0) vf[er[r]] = l;
        } else {
          gl = l;
        }
      }
    }
  }
  __builtin_amdgcn_wave_barrier();
  // 5. the picks ranked (ties to the lower index), softmax scores as topk_wave forms them over v, the folded shared
  // expert's slots
  float v[NPL];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int e = lane + 64 * j;
    v[j] = vf[min(e, E - 1)];
    if (e < E) {
      mx = fmaxf(mx, v[j]);
      if (a.logits) a.logits[size_t(t) * E + e] = v[j];
    }
  }
  const int ks = a.k + a.m;
  if (lane == 0) {
    if (a.gate && a.wsg) a.gate[t] = gl;
    if (a.n_cand) a.n_cand[t] = n;
  }
  uint32_t id;
  float sc;
  if (all) {  // every expert's logit is the fixed-order one: the wave top-k over all of them
    topk_wave<NPL, true>(v, E, a.k, a.norm, scr[wave], &id, &sc);
  } else {
    mx = wave_max(mx);
    float se = 0.0f;
#pragma unroll
    for (int j = 0; j < NPL; ++j)
      if (lane + 64 * j < E) se += __expf(v[j] - mx);
    se = wave_sum(se);
    const uint32_t my_idx = lane < n ? cidx[wave][lane] : 0u;
    const uint32_t my_key = lane < n ? logit_key(vf[my_idx]) : 0u;
    if (lane < n) ckey[wave][lane] = my_key;
    __builtin_amdgcn_wave_barrier();
    int rank = 64;
    if (lane < n) {
      rank = 0;
      for (int o = 0; o < n; ++o) {
        const uint32_t ko = ckey[wave][o], io = cidx[wave][o];
        rank += (ko > my_key || (ko == my_key && io < my_idx)) ? 1 : 0;
      }
    }
    // lane r < k takes the rank-r pick (ranks are distinct)
    uint32_t pid = 0xFFFFFFFFu, pkey = 0;
    for (int r = 0; r < a.k; ++r) {
      const uint64_t hit = __ballot(rank == r);
      const int src = hit ? __builtin_ctzll(hit) : 0;
      const uint32_t i_r = uint32_t(__builtin_amdgcn_readlane(int(my_idx), src));
      const uint32_t k_r = uint32_t(__builtin_amdgcn_readlane(int(my_key), src));
      if (lane == r) {
        pid = hit ? i_r : 0xFFFFFFFFu;
        pkey = k_r;
      }
    }
    id = pid;
    float mine = lane < a.k ? __expf(key_logit(pkey) - mx) / se : 0.0f;
    if (a.norm) {
      float tot = 0.0f;  // the k picked probabilities summed in rank order
      for (int r = 0; r < a.k; ++r)
        tot += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mine), r));
      mine = mine / tot;
    }
    sc = mine;
  }
  if (lane < a.k) {
    a.ids[size_t(t) * ks + lane] = id;
    a.scores[size_t(t) * ks + lane] = sc;
  } else if (lane < ks) {
    a.ids[size_t(t) * ks + lane] = uint32_t(E + lane - a.k);
    a.scores[size_t(t) * ks + lane] = sigmoidf_(gl);
  }
}

}  // namespace lmoe

using namespace lmoe;

extern "C" int lmoe_router_norms(const void *wr, const void *wsg, int wdtype, int E, int H, float *norms,
                                 void *stream) {
  static const char *fn = "lmoe_router_norms";
  LMOE_REQUIRE(dtype_ok(wdtype), LMOE_EINVAL, "%s: bad dtype", fn);
  LMOE_REQUIRE(E > 0 && E <= rf::kMaxE && H > 0, LMOE_ESHAPE, "%s: %d rows of %d", fn, E, H);
  LMOE_REQUIRE(wr && norms, LMOE_EINVAL, "%s: null pointer", fn);
  launch(k_router_norms, dim3(unsigned(E + (wsg ? 1 : 0))), dim3(256), 0, static_cast<hipStream_t>(stream), wr, wsg,
         wdtype, E, H, norms);
  LMOE_LAUNCHED(fn);
  return 0;
}

extern "C" int lmoe_router_refine(const float *part, int ksplit, int ldp, const void *x, int xdtype, int T, int H,
                                  const void *wr, const void *wsg, int wdtype, int E, const float *norms, int k,
                                  int norm, int m, uint32_t *ids, float *scores, float *logits, float *gate,
                                  int *n_cand, void *stream) {
  static const char *fn = "lmoe_router_refine";
  LMOE_REQUIRE(dtype_ok(xdtype) && dtype_ok(wdtype), LMOE_EINVAL, "%s: bad dtype", fn);
  LMOE_REQUIRE(T >= 0 && H > 0 && H % 8 == 0 && H <= rf::kMaxH, LMOE_ESHAPE, "%s: hidden %d (a multiple of 8, at most "
               "%d)", fn, H, rf::kMaxH);
  LMOE_REQUIRE(E > 0 && E <= rf::kMaxE && k > 0 && k <= E && k <= 32 && m >= 0 && k + m <= 64, LMOE_ESHAPE,
               "%s: top-%d of %d experts with %d shared slices", fn, k, E, m);
  LMOE_REQUIRE(ksplit == 1 || ksplit == 2 || ksplit == 4 || ksplit == 8, LMOE_ESHAPE, "%s: K split %d", fn, ksplit);
  LMOE_REQUIRE(ldp >= E, LMOE_ESHAPE, "%s: row stride %d", fn, ldp);  // only the E experts' columns are read
  LMOE_REQUIRE(m == 0 || wsg, LMOE_EINVAL, "%s: shared slices need the gate row", fn);
  if (T == 0) return 0;
  LMOE_REQUIRE(part && x && wr && norms && ids && scores, LMOE_EINVAL, "%s: null pointer", fn);
  LMOE_REQUIRE(aligned16(wr) && (!wsg || aligned16(wsg)) && aligned16(norms), LMOE_EALIGN,
               "%s: router weights and norms must be 16-byte aligned", fn);
  RefineArgs a{};
  a.part = part, a.ks = ksplit, a.ldp = ldp, a.x = x, a.xdt = xdtype, a.T = T, a.H = H, a.wr = wr, a.wsg = wsg;
  a.wdt = wdtype, a.E = E, a.norms = norms, a.k = k, a.norm = norm, a.m = m, a.ids = ids, a.scores = scores;
  a.logits = logits, a.gate = gate, a.n_cand = n_cand;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int xcn = (H / 8 + rf::NT - 1) / rf::NT;
  const size_t lds = size_t(4) * (4 * ((E + 3) & ~3) + H * (xdtype == LMOE_F32 ? 4 : 2));
  LMOE_REQUIRE(lds <= 160 * 1024, LMOE_ESHAPE, "%s: %zu bytes of LDS", fn, lds);
  int rc = 0;
  auto go4 = [&](auto npl, auto ksc, auto xcc) {
    constexpr int N = decltype(npl)::value, K = decltype(ksc)::value, X = decltype(xcc)::value;
    auto kern = wdtype == LMOE_F16    ? k_router_refine<N, LMOE_F16, K, X>
                : wdtype == LMOE_BF16 ? k_router_refine<N, LMOE_BF16, K, X>
                                      : k_router_refine<N, LMOE_F32, K, X>;
    rc = allow_lds(kern, lds, fn);
    if (rc == 0) launch(kern, dim3(unsigned((T + 3) / 4)), dim3(rf::NT), lds, st, a);
  };
  auto go3 = [&](auto npl, auto ksc) {
    if (xcn <= 1) go4(npl, ksc, std::integral_constant<int, 1>());
    else if (xcn <= 2) go4(npl, ksc, std::integral_constant<int, 2>());
    else go4(npl, ksc, std::integral_constant<int, 4>());
  };
  auto go = [&](auto npl) {
    if (ksplit == 1) go3(npl, std::integral_constant<int, 1>());
    else if (ksplit == 2) go3(npl, std::integral_constant<int, 2>());
    else if (ksplit == 4) go3(npl, std::integral_constant<int, 4>());
    else go3(npl, std::integral_constant<int, 8>());
  };
  if (E <= 64) go(std::integral_constant<int, 1>());
  else if (E <= 128) go(std::integral_constant<int, 2>());
  else if (E <= 256) go(std::integral_constant<int, 4>());
  else if (E <= 512) go(std::integral_constant<int, 8>());
  else go(std::integral_constant<int, 16>());
  if (rc) return rc;
  LMOE_LAUNCHED(fn);
  return 0;
}
