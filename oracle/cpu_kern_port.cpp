// CPU baseline: a standalone restatement of the reference CPU kernel's expert gather-matmul
// (cpu_ext/cpu_kern.cpp: rows_kernel :87-154, prep_x :159-186, run_jobs :200-227, the gather job split
// :300-349), without MLX or nanobind, plus converters from GGUF Q4_0 / Q4_K to the affine 4-bit layout it reads
// and a MoE-layer harness (router, top-k, gate/up, SwiGLU, down, combine) so a whole layer can be timed.
//
// TEST INFRASTRUCTURE ONLY: this is the CPU baseline that bench.py times beside the GPU and that the tests check
// against float64; the product path never loads it.
//
// Affine 4-bit (MLX's packing): weight i of a row sits in bits 4 (i mod 8) of 32-bit word i / 8; group g of gs
// weights has a scale s_g and bias b_g; w = s_g q + b_g. The kernel computes, per output row,
//   y = sum_g s_g * dot(x_g, q_g) + sum_g b_g * sum(x_g)
// with x rearranged per 32-chunk as [16 even k, 16 odd k] (the low and high nibbles of 16 bytes), f32 FMAs into
// 16-wide accumulators, MB = 8 x rows a pass reusing each unpacked weight chunk, and OpenMP dynamic scheduling over
// row chunks of max(8, min(64, N / 8)) rows. A Q4_0 block maps losslessly onto a group of 32 (s = d, b = -8 d);
// a Q4_K sub-block onto a group of 32 (s = d * sc, b = -dmin * m), both exact in f32. With gs = 32 the
// reference takes its f32 path (the bf16 dot-product path needs gs % 64 == 0, cpu_kern.cpp:328).
#include <immintrin.h>
#include <omp.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

namespace {

int g_threads = 1;
constexpr int MB = 8;

inline float f16_to_f32(uint16_t h) {
  const uint32_t s = uint32_t(h & 0x8000u) << 16, e = (h >> 10) & 0x1F, m = h & 0x3FF;
  uint32_t u;
  if (e == 0) {
    if (m == 0) {
      u = s;
    } else {  // subnormal: normalise
      int ee = -1;
      uint32_t mm = m;
      do {
        ++ee;
        mm <<= 1;
      } while (!(mm & 0x400));
      u = s | uint32_t(127 - 15 - ee) << 23 | (mm & 0x3FF) << 13;
    }
  } else if (e == 31) {
    u = s | 0x7F800000u | m << 13;
  } else {
    u = s | (e + 112) << 23 | m << 13;
  }
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// ---- the row kernel: AVX-512 f32 path, and a portable scalar twin for hosts without AVX-512 ------------------

__attribute__((target("avx512f,avx512bw"))) void rows_avx512(const uint8_t *w, const float *sc, const float *bi,
                                                              int K, int gs, int n0, int n1, int M,
                                                              const float *const *xp, const float *const *xs,
                                                              float *const *yp) {
  const int G = K / gs;
  const size_t rb = size_t(K) / 2;
  const __m512i m0f = _mm512_set1_epi32(0x0f);
  for (int n = n0; n < n1; ++n) {
    const uint8_t *wr = w + size_t(n) * rb;
    const float *sf = sc + size_t(n) * G, *bf = bi + size_t(n) * G;
    for (int m0 = 0; m0 < M; m0 += MB) {
      const int mb = std::min(MB, M - m0);
      __m512 acc[MB];
      for (int i = 0; i < MB; ++i) acc[i] = _mm512_setzero_ps();
      for (int g = 0; g < G; ++g) {
        __m512 t[MB];
        for (int i = 0; i < MB; ++i) t[i] = _mm512_setzero_ps();
        const int k0 = g * gs;
        for (int c = 0; c < gs; c += 32) {
          const __m512i d = _mm512_cvtepu8_epi32(_mm_loadu_si128(reinterpret_cast<const __m128i *>(wr + (k0 + c) / 2)));
          const __m512 lo = _mm512_cvtepi32_ps(_mm512_and_si512(d, m0f));
          const __m512 hi = _mm512_cvtepi32_ps(_mm512_srli_epi32(d, 4));
          for (int i = 0; i < mb; ++i) {
            const float *x = xp[m0 + i] + k0 + c;
            t[i] = _mm512_fmadd_ps(lo, _mm512_loadu_ps(x), t[i]);
            t[i] = _mm512_fmadd_ps(hi, _mm512_loadu_ps(x + 16), t[i]);
          }
        }
        const __m512 s = _mm512_set1_ps(sf[g]);
        for (int i = 0; i < mb; ++i) acc[i] = _mm512_fmadd_ps(t[i], s, acc[i]);
      }
      for (int i = 0; i < mb; ++i) {
        float b = 0.f;
        for (int g = 0; g < G; ++g) b += bf[g] * xs[m0 + i][g];
        yp[m0 + i][n] = _mm512_reduce_add_ps(acc[i]) + b;
      }
    }
  }
}

void rows_scalar(const uint8_t *w, const float *sc, const float *bi, int K, int gs, int n0, int n1, int M,
                 const float *const *xp, const float *const *xs, float *const *yp) {
  const int G = K / gs;
  const size_t rb = size_t(K) / 2;
  for (int n = n0; n < n1; ++n) {
    const uint8_t *wr = w + size_t(n) * rb;
    for (int i = 0; i < M; ++i) {
      float acc = 0.f, b = 0.f;
      for (int g = 0; g < G; ++g) {
        float t = 0.f;
        const int k0 = g * gs;
        for (int c = 0; c < gs; c += 32)
          for (int j = 0; j < 16; ++j) {
            const uint8_t v = wr[(k0 + c) / 2 + j];
            t = std::fma(float(v & 15), xp[i][k0 + c + j], t);
            t = std::fma(float(v >> 4), xp[i][k0 + c + 16 + j], t);
          }
        acc = std::fma(t, sc[size_t(n) * G + g], acc);
        b += bi[size_t(n) * G + g] * xs[i][g];
      }
      yp[i][n] = acc + b;
    }
  }
}

bool has_avx512() { return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw"); }

// x row into the kernel layout: each 32-chunk as [16 even k, 16 odd k]; plus the group sums.
void prep_x(const float *x, int K, int gs, float *out, float *sums) {
  for (int c = 0; c < K; c += 32)
    for (int j = 0; j < 16; ++j) {
      out[c + j] = x[c + 2 * j];
      out[c + 16 + j] = x[c + 2 * j + 1];
    }
  for (int g = 0; g < K / gs; ++g) {
    float s = 0.f;
    for (int k = g * gs; k < (g + 1) * gs; ++k) s += x[k];
    sums[g] = s;
  }
}

struct Job {
  const uint8_t *w;
  const float *sc, *bi;
  std::vector<const float *> xp, xs;
  std::vector<float *> yp;
};

void run_jobs(std::vector<Job> &jobs, int N, int K, int gs) {
  const int chunk = std::max(8, std::min(64, N / 8));
  struct Task {
    int j, n0, n1;
  };
  std::vector<Task> tasks;
  for (int j = 0; j < int(jobs.size()); ++j)
    for (int n = 0; n < N; n += chunk) tasks.push_back({j, n, std::min(N, n + chunk)});
  const bool v = has_avx512();
  auto one = [&](int i) {
    const Task &t = tasks[i];
    Job &jb = jobs[t.j];
    const int M = int(jb.xp.size());
    if (v)
      rows_avx512(jb.w, jb.sc, jb.bi, K, gs, t.n0, t.n1, M, jb.xp.data(), jb.xs.data(), jb.yp.data());
    else
      rows_scalar(jb.w, jb.sc, jb.bi, K, gs, t.n0, t.n1, M, jb.xp.data(), jb.xs.data(), jb.yp.data());
  };
  const int nt = int(tasks.size());
  if (nt == 1 || g_threads == 1) {
    for (int i = 0; i < nt; ++i) one(i);
    return;
  }
#pragma omp parallel for schedule(dynamic, 1) num_threads(g_threads)
  for (int i = 0; i < nt; ++i) one(i);
}

}  // namespace

extern "C" {

int ckp_set_threads(int n) {
  g_threads = n > 0 ? n : 1;
  return g_threads;
}

int ckp_has_avx512(void) { return has_avx512() ? 1 : 0; }

// y[r] = x[r] . W[idx[r]]^T for R rows: x [R][K] f32, w uint8 [E][N][K / 2] (MLX nibble order), sc/bi f32
// [E][N][K / gs], y [R][N] f32. idx >= E gives zero rows (cpu_kern.cpp:316-318).
int ckp_gather_qmm(const float *x, int R, int K, const uint8_t *w, const float *sc, const float *bi, int E, int N,
                   int gs, const uint32_t *idx, float *y) {
  if (K % gs || gs % 32 || K % 32) return -1;
  const int G = K / gs;
  const size_t wbytes = size_t(N) * K / 2, sbytes = size_t(N) * G;
  std::vector<float> xb(size_t(R) * K), sb(size_t(R) * G);
  auto prep = [&](int r) { prep_x(x + size_t(r) * K, K, gs, xb.data() + size_t(r) * K, sb.data() + size_t(r) * G); };
  if (R >= 64) {
#pragma omp parallel for num_threads(g_threads)
    for (int r = 0; r < R; ++r) prep(r);
  } else {
    for (int r = 0; r < R; ++r) prep(r);
  }
  std::vector<Job> jobs;
  std::vector<int> job_of(E, -1);
  for (int r = 0; r < R; ++r) {
    const uint32_t e = idx[r];
    if (e >= uint32_t(E)) {
      std::memset(y + size_t(r) * N, 0, size_t(N) * 4);
      continue;
    }
    if (job_of[e] < 0) {
      job_of[e] = int(jobs.size());
      jobs.push_back(Job{w + e * wbytes, sc + e * sbytes, bi + e * sbytes, {}, {}, {}});
    }
    Job &jb = jobs[job_of[e]];
    jb.xp.push_back(xb.data() + size_t(r) * K);
    jb.xs.push_back(sb.data() + size_t(r) * G);
    jb.yp.push_back(y + size_t(r) * N);
  }
  run_jobs(jobs, N, K, gs);
  return 0;
}

// GGUF Q4_0 rows (rows x K / 32 blocks of 18 bytes) -> affine gs 32: w [rows][K / 2], sc = d, bi = -8 d.
int ckp_q4_0_to_affine(const uint8_t *q, long long rows, int K, uint8_t *w, float *sc, float *bi) {
  if (K % 32) return -1;
  const int nb = K / 32;
#pragma omp parallel for num_threads(g_threads)
  for (long long r = 0; r < rows; ++r) {
    for (int b = 0; b < nb; ++b) {
      const uint8_t *blk = q + (size_t(r) * nb + b) * 18;
      const float d = f16_to_f32(uint16_t(blk[0] | blk[1] << 8));
      uint8_t e[32];
      for (int j = 0; j < 16; ++j) {
        e[j] = blk[2 + j] & 15;
        e[j + 16] = blk[2 + j] >> 4;
      }
      uint8_t *o = w + size_t(r) * (K / 2) + 16 * b;
      for (int m = 0; m < 16; ++m) o[m] = uint8_t(e[2 * m] | e[2 * m + 1] << 4);
      sc[size_t(r) * nb + b] = d;
      bi[size_t(r) * nb + b] = -8.0f * d;
    }
  }
  return 0;
}

// GGUF Q4_K rows (rows x K / 256 super-blocks of 144 bytes) -> affine gs 32: sc = d sc_j, bi = -dmin m_j.
int ckp_q4_k_to_affine(const uint8_t *q, long long rows, int K, uint8_t *w, float *sc, float *bi) {
  if (K % 256) return -1;
  const int ns = K / 256;
#pragma omp parallel for num_threads(g_threads)
  for (long long r = 0; r < rows; ++r) {
    for (int s = 0; s < ns; ++s) {
      const uint8_t *b = q + (size_t(r) * ns + s) * 144;
      const float d = f16_to_f32(uint16_t(b[0] | b[1] << 8)), dmin = f16_to_f32(uint16_t(b[2] | b[3] << 8));
      const uint8_t *k = b + 4;
      for (int j = 0; j < 8; ++j) {
        int scj, mj;
        if (j < 4) {
          scj = k[j] & 63;
          mj = k[j + 4] & 63;
        } else {
          scj = (k[j + 4] & 15) | ((k[j - 4] >> 6) << 4);
          mj = (k[j + 4] >> 4) | ((k[j] >> 6) << 4);
        }
        const size_t g = size_t(r) * (K / 32) + 8 * s + j;
        sc[g] = d * float(scj);
        bi[g] = -(dmin * float(mj));
        const uint8_t *qs = b + 16 + 32 * (j / 2);
        uint8_t e[32];
        for (int l = 0; l < 32; ++l) e[l] = (j & 1) ? (qs[l] >> 4) : (qs[l] & 15);
        uint8_t *o = w + size_t(r) * (K / 2) + 16 * (8 * s + j);
        for (int m = 0; m < 16; ++m) o[m] = uint8_t(e[2 * m] | e[2 * m + 1] << 4);
      }
    }
  }
  return 0;
}

// One MoE layer on T tokens, end to end on the CPU: logits = x . wr (f16 weights, f32 sums), top-k with ties to
// the lowest index, softmax scores (renormalised when norm), gate/up/down through ckp_gather_qmm on the affine
// experts (gs 32), SwiGLU, the weighted combine and a residual add (residual may be null). x, out [T][H] f32.
int ckp_moe_layer(const float *x, int T, int H, const uint16_t *wr, int E, int k, int norm, int I,
                  const uint8_t *gw, const float *gs_, const float *gb, const uint8_t *uw, const float *us,
                  const float *ub, const uint8_t *dw, const float *ds, const float *db, const float *residual,
                  float *out) {
  std::vector<uint32_t> idx(size_t(T) * k);
  std::vector<float> score(size_t(T) * k);
  std::vector<float> lg(E);
  for (int t = 0; t < T; ++t) {
    const float *xt = x + size_t(t) * H;
    for (int e = 0; e < E; ++e) {
      float s = 0.f;
      const uint16_t *we = wr + size_t(e) * H;
      for (int h = 0; h < H; ++h) s += xt[h] * f16_to_f32(we[h]);
      lg[e] = s;
    }
    const float mx = *std::max_element(lg.begin(), lg.end());
    float tot = 0.f;
    for (int e = 0; e < E; ++e) tot += std::exp(lg[e] - mx);
    std::vector<int> ord(E);
    for (int e = 0; e < E; ++e) ord[e] = e;
    std::partial_sort(ord.begin(), ord.begin() + k, ord.end(),
                      [&](int a, int b) { return lg[a] > lg[b] || (lg[a] == lg[b] && a < b); });
    float ks = 0.f;
    for (int j = 0; j < k; ++j) {
      idx[size_t(t) * k + j] = uint32_t(ord[j]);
      score[size_t(t) * k + j] = std::exp(lg[ord[j]] - mx) / tot;
      ks += score[size_t(t) * k + j];
    }
    if (norm)
      for (int j = 0; j < k; ++j) score[size_t(t) * k + j] /= ks;
  }
  const int R = T * k;
  std::vector<float> xr(size_t(R) * H), g(size_t(R) * I), u(size_t(R) * I), y(size_t(R) * H);
  for (int r = 0; r < R; ++r) std::memcpy(xr.data() + size_t(r) * H, x + size_t(r / k) * H, size_t(H) * 4);
  ckp_gather_qmm(xr.data(), R, H, gw, gs_, gb, E, I, 32, idx.data(), g.data());
  ckp_gather_qmm(xr.data(), R, H, uw, us, ub, E, I, 32, idx.data(), u.data());
  for (size_t i = 0; i < g.size(); ++i) g[i] = g[i] / (1.f + std::exp(-g[i])) * u[i];
  ckp_gather_qmm(g.data(), R, I, dw, ds, db, E, H, 32, idx.data(), y.data());
  for (int t = 0; t < T; ++t)
    for (int h = 0; h < H; ++h) {
      float a = residual ? residual[size_t(t) * H + h] : 0.f;
      for (int j = 0; j < k; ++j) a += score[size_t(t) * k + j] * y[(size_t(t) * k + j) * H + h];
      out[size_t(t) * H + h] = a;
    }
  return 0;
}

}  // extern "C"
