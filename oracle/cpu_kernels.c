/*
 * ORACLE (test infrastructure only) - C restatement of the reference's CPU kernels for the
 * quantized decode path, with the same algorithms and the same OpenMP work decomposition:
 *
 *   oracle_int8_linear        int8_linear,  reference src/llmserve/kernels/csrc/int8_gemv.cpp:13-46
 *   oracle_int4_linear        int4_linear,  int8_gemv.cpp:53-107 (serial per-group x sums,
 *                             then rows in parallel; s * sum(x q) + (z - 8 s) * sum(x))
 *   oracle_paged_decode_int8  paged_attention_decode_int8 -> pa2::decode<int8_t>,
 *                             paged_attention.cpp:141-346 and :361-376 (partition heuristic,
 *                             online softmax per block of tokens, merge of partitions)
 *
 * Built with the reference's flags (-O3 -march=<isa> -fopenmp -ffast-math,
 * kernels/__init__.py:58-72). Pinned by tests/test_oracle_cpu.py against the float64
 * mathematics of oracle/math_ref.py at the reference tests' tolerances and, when built,
 * against the reference's own compiled kernels in oracle/_ref/.
 * Used by tests/ as the parity checker of the HIP kernels and by bench.py as the timed
 * CPU baseline; never by the product.
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* at::parallel_for(0, n, grain): contiguous ranges, one per thread, of at least `grain`. */
static int64_t chunk_count(int64_t n, int64_t grain) {
  int64_t t = omp_get_max_threads();
  int64_t by_grain = (n + grain - 1) / grain;
  return t < by_grain ? t : by_grain;
}

void oracle_int8_linear(const float* x, const int8_t* q, const float* scale, float* y,
                        int64_t M, int64_t N, int64_t K) {
  const int64_t chunks = chunk_count(N, 64);
  if (chunks <= 0) return;
  const int64_t per = (N + chunks - 1) / chunks;
#pragma omp parallel for schedule(static)
  for (int64_t c = 0; c < chunks; ++c) {
    float acc[64];
    const int64_t n1 = (c + 1) * per < N ? (c + 1) * per : N;
    for (int64_t n = c * per; n < n1; ++n) {
      const int8_t* w = q + n * K;
      for (int64_t m = 0; m < M; ++m) {
        const float* xr = x + m * K;
        float s = 0.f;
#pragma omp simd reduction(+ : s)
        for (int64_t k = 0; k < K; ++k) s += xr[k] * (float)w[k];
        acc[m] = s;
      }
      const float sc = scale[n];
      for (int64_t m = 0; m < M; ++m) y[m * N + n] = acc[m] * sc;
    }
  }
}

void oracle_int4_linear(const float* x, const uint8_t* nib, const float* gs, const float* gz,
                        float* y, int64_t M, int64_t N, int64_t K, int64_t group) {
  const int64_t G = K / group, half = group / 2;
  float* xsum = (float*)malloc(sizeof(float) * (size_t)(M * G > 0 ? M * G : 1));
  for (int64_t m = 0; m < M; ++m)
    for (int64_t g = 0; g < G; ++g) {
      const float* xr = x + m * K + g * group;
      float s = 0.f;
#pragma omp simd reduction(+ : s)
      for (int64_t k = 0; k < group; ++k) s += xr[k];
      xsum[m * G + g] = s;
    }
  const int64_t chunks = chunk_count(N, 64);
  const int64_t per = chunks > 0 ? (N + chunks - 1) / chunks : 0;
#pragma omp parallel for schedule(static)
  for (int64_t c = 0; c < chunks; ++c) {
    const int64_t n1 = (c + 1) * per < N ? (c + 1) * per : N;
    for (int64_t n = c * per; n < n1; ++n) {
      const uint8_t* row = nib + n * (K / 2);
      for (int64_t m = 0; m < M; ++m) {
        const float* xr = x + m * K;
        float total = 0.f;
        for (int64_t g = 0; g < G; ++g) {
          const uint8_t* b = row + g * half;
          const float* xg = xr + g * group;
          float d = 0.f;
#pragma omp simd reduction(+ : d)
          for (int64_t j = 0; j < half; ++j)
            d += xg[2 * j] * (float)(b[j] & 0xF) + xg[2 * j + 1] * (float)(b[j] >> 4);
          const float s = gs[n * G + g], z = gz[n * G + g];
          total += s * d + (z - 8.f * s) * xsum[m * G + g];
        }
        y[m * N + n] = total;
      }
    }
  }
  free(xsum);
}

/* Online-softmax attention of G query heads over cache tokens [t0, t1) of one
 * (sequence, kv head); acc [G, D] unnormalised, m running max, l running sum. */
static void attend_range_i8(const float* qg, const int8_t* kc, const int8_t* vc,
                            const float* ks, const float* vs, const int64_t* bt, int64_t t0,
                            int64_t t1, int64_t bs, int64_t Hk, int64_t h, int64_t G, int64_t D,
                            float scale, float* acc, float* m, float* l, float* sc) {
  for (int64_t g = 0; g < G; ++g) {
    m[g] = -1e30f;
    l[g] = 0.f;
  }
  memset(acc, 0, sizeof(float) * (size_t)(G * D));
  const int64_t row = Hk * D;
  for (int64_t t = t0; t < t1;) {
    const int64_t off = t % bs;
    const int64_t n = (bs - off) < (t1 - t) ? (bs - off) : (t1 - t);
    const int64_t slot0 = bt[t / bs] * bs + off;
    for (int64_t j = 0; j < n; ++j) {
      const int64_t slot = slot0 + j;
      const int8_t* kt = kc + slot * row + h * D;
      const float f = scale * ks[slot * Hk + h];
      for (int64_t g = 0; g < G; ++g) {
        const float* qq = qg + g * D;
        float d = 0.f;
#pragma omp simd reduction(+ : d)
        for (int64_t i = 0; i < D; ++i) d += qq[i] * (float)kt[i];
        sc[g * bs + j] = f * d;
      }
    }
    for (int64_t g = 0; g < G; ++g) {
      float* s = sc + g * bs;
      float mb = m[g];
      for (int64_t j = 0; j < n; ++j) mb = s[j] > mb ? s[j] : mb;
      const float alpha = expf(m[g] - mb);
      if (alpha != 1.f) {
        float* a = acc + g * D;
        for (int64_t i = 0; i < D; ++i) a[i] *= alpha;
      }
      float sum = 0.f;
      for (int64_t j = 0; j < n; ++j) {
        s[j] = expf(s[j] - mb);
        sum += s[j];
      }
      l[g] = l[g] * alpha + sum;
      m[g] = mb;
    }
    for (int64_t j = 0; j < n; ++j) {
      const int64_t slot = slot0 + j;
      const int8_t* vt = vc + slot * row + h * D;
      const float vsc = vs[slot * Hk + h];
      for (int64_t g = 0; g < G; ++g) {
        const float w = sc[g * bs + j] * vsc;
        float* a = acc + g * D;
#pragma omp simd
        for (int64_t i = 0; i < D; ++i) a[i] += w * (float)vt[i];
      }
    }
    t += n;
  }
}

/* Returns the partition size used (tokens), or -1 on bad arguments. */
int64_t oracle_paged_decode_int8(const float* q, const int8_t* kc, const int8_t* vc,
                                 const float* ks, const float* vs, const int64_t* bt,
                                 const int64_t* cl, float* out, int64_t B, int64_t Hq, int64_t Hk,
                                 int64_t D, int64_t max_blocks, int64_t bs, float scale,
                                 int64_t partition_size) {
  if (B <= 0) return 0;
  if (Hk <= 0 || Hq % Hk) return -1;
  const int64_t G = Hq / Hk;
  int64_t max_ctx = 1;
  for (int64_t b = 0; b < B; ++b) max_ctx = cl[b] > max_ctx ? cl[b] : max_ctx;
  int64_t P = partition_size;
  if (P <= 0) {
    const int64_t want = 4 * (int64_t)omp_get_max_threads();
    int64_t parts = (want + B * Hk - 1) / (B * Hk);
    if (parts < 1) parts = 1;
    P = (max_ctx + parts - 1) / parts;
    if (P < 2 * bs) P = 2 * bs;
  }
  P = ((P + bs - 1) / bs) * bs;
  const int64_t NP = (max_ctx + P - 1) / P;
  const int64_t items = B * Hk * NP;
  float *pacc = NULL, *pm = NULL, *pl = NULL;
  if (NP > 1) {
    pacc = (float*)malloc(sizeof(float) * (size_t)(items * G * D));
    pm = (float*)malloc(sizeof(float) * (size_t)(items * G));
    pl = (float*)malloc(sizeof(float) * (size_t)(items * G));
  }
#pragma omp parallel
  {
    float* sc = (float*)malloc(sizeof(float) * (size_t)(G * bs));
    float* m = (float*)malloc(sizeof(float) * (size_t)G);
    float* l = (float*)malloc(sizeof(float) * (size_t)G);
    float* acc = (float*)malloc(sizeof(float) * (size_t)(G * D));
#pragma omp for schedule(static)
    for (int64_t idx = 0; idx < items; ++idx) {
      const int64_t p = idx % NP, bh = idx / NP, b = bh / Hk, h = bh % Hk;
      const int64_t ctx = cl[b];
      const int64_t t0 = p * P, t1 = ctx < t0 + P ? ctx : t0 + P;
      const float* qb = q + (b * Hq + h * G) * D;
      const int64_t* btb = bt + b * max_blocks;
      if (NP == 1) {
        attend_range_i8(qb, kc, vc, ks, vs, btb, t0, t1, bs, Hk, h, G, D, scale, acc, m, l, sc);
        float* ob = out + (b * Hq + h * G) * D;
        for (int64_t g = 0; g < G; ++g) {
          const float inv = 1.f / l[g];
          for (int64_t i = 0; i < D; ++i) ob[g * D + i] = acc[g * D + i] * inv;
        }
        continue;
      }
      if (t0 >= t1) {
        for (int64_t g = 0; g < G; ++g) {
          pm[idx * G + g] = -1e30f;
          pl[idx * G + g] = 0.f;
        }
        continue;
      }
      attend_range_i8(qb, kc, vc, ks, vs, btb, t0, t1, bs, Hk, h, G, D, scale,
                      pacc + idx * G * D, pm + idx * G, pl + idx * G, sc);
    }
    free(sc);
    free(m);
    free(l);
    free(acc);
  }
  if (NP > 1) {
#pragma omp parallel for schedule(static)
    for (int64_t bh = 0; bh < B * Hk; ++bh) {
      const int64_t b = bh / Hk, h = bh % Hk;
      float* ob = out + (b * Hq + h * G) * D;
      for (int64_t g = 0; g < G; ++g) {
        float Mx = -1e30f;
        for (int64_t p = 0; p < NP; ++p) {
          const float v = pm[(bh * NP + p) * G + g];
          Mx = v > Mx ? v : Mx;
        }
        float L = 0.f;
        float* o = ob + g * D;
        memset(o, 0, sizeof(float) * (size_t)D);
        for (int64_t p = 0; p < NP; ++p) {
          const int64_t i = (bh * NP + p) * G + g;
          if (pl[i] == 0.f) continue;
          const float w = expf(pm[i] - Mx);
          L += w * pl[i];
          const float* a = pacc + i * D;
          for (int64_t d = 0; d < D; ++d) o[d] += w * a[d];
        }
        const float inv = 1.f / L;
        for (int64_t d = 0; d < D; ++d) o[d] *= inv;
      }
    }
    free(pacc);
    free(pm);
    free(pl);
  }
  return P;
}

void oracle_set_threads(int n) {
  if (n > 0) omp_set_num_threads(n);
}

int oracle_get_threads(void) { return omp_get_max_threads(); }
