/*
 * CPU oracle, C restatement -- TEST INFRASTRUCTURE ONLY.
 *
 * Used by tests/ (large parity cases where the numpy loop would be slow) and
 * by the cpu_baseline leg of bench.py.  The product library never links it.
 *
 * It restates the reference's per-token KDA recurrence
 * (Arain119/Sophia ml/runtime/model/attention.py:260-294, _reference_kda)
 * over a packed ragged batch (the cu_seqlens contract of
 * ml/training/pretrain/engine/sm120_concurrent_ffn.py:209-268): state resets
 * to the given initial state (or zero) at every sequence boundary.
 * fp32 arithmetic throughout, like the reference's CPU run.  OpenMP spreads
 * the independent (sequence, head) pairs over threads.
 *
 * Parity: pinned against oracle/kda_oracle.py (numpy) on seeded inputs, which
 * is itself pinned against closed forms (tests/test_oracle_kda.py).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORACLE_QK_L2NORM 1
#define ORACLE_GATE 2
#define ORACLE_BETA_SIGMOID 4

static float sigmoidf_ref(float x) { return 1.0f / (1.0f + expf(-x)); }

/* q, k, g: [T, H, K]; v, o: [T, H, V]; beta: [T, H]; h0, ht: [N, H, K, V]. */
int oracle_kda_varlen_f32(const float *q, const float *k, const float *v, const float *g,
                          const float *beta, const float *A_log, const float *dt_bias,
                          float lower_bound, float scale, int flags, const int32_t *cu_seqlens,
                          int n_seqs, int H, int K, int V, const float *h0, float *o, float *ht,
                          int nthreads) {
  if (K <= 0 || V <= 0 || H <= 0 || n_seqs < 0) return -1;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#else
  (void)nthreads;
#endif
  const long pairs = (long)n_seqs * H;
  int bad = 0;
#pragma omp parallel for schedule(dynamic, 1)
  for (long p = 0; p < pairs; ++p) {
    const int s = (int)(p / H), h = (int)(p % H);
    float *S = (float *)malloc(sizeof(float) * (size_t)K * V);
    float *qn = (float *)malloc(sizeof(float) * (size_t)K);
    float *kn = (float *)malloc(sizeof(float) * (size_t)K);
    float *al = (float *)malloc(sizeof(float) * (size_t)K);
    float *pred = (float *)malloc(sizeof(float) * (size_t)V);
    float *acc = (float *)malloc(sizeof(float) * (size_t)V);
    if (!S || !qn || !kn || !al || !pred || !acc) {
#pragma omp atomic write
      bad = 1;
      free(S); free(qn); free(kn); free(al); free(pred); free(acc);
      continue;
    }
    const size_t soff = ((size_t)s * H + h) * (size_t)K * V;
    if (h0)
      memcpy(S, h0 + soff, sizeof(float) * (size_t)K * V);
    else
      memset(S, 0, sizeof(float) * (size_t)K * V);
    const float head_scale = A_log ? expf(A_log[h]) : 1.0f;
    for (int t = cu_seqlens[s]; t < cu_seqlens[s + 1]; ++t) {
      const float *qt = q + ((size_t)t * H + h) * K;
      const float *kt = k + ((size_t)t * H + h) * K;
      const float *gt = g + ((size_t)t * H + h) * K;
      const float *vt = v + ((size_t)t * H + h) * V;
      float qs = 1.0f, ks = 1.0f;
      if (flags & ORACLE_QK_L2NORM) {
        float sq = 0.f, sk = 0.f;
        for (int i = 0; i < K; ++i) { sq += qt[i] * qt[i]; sk += kt[i] * kt[i]; }
        qs = 1.0f / fmaxf(sqrtf(sq), 1e-12f);
        ks = 1.0f / fmaxf(sqrtf(sk), 1e-12f);
      }
      for (int i = 0; i < K; ++i) {
        qn[i] = qt[i] * qs * scale;
        kn[i] = kt[i] * ks;
        float gl = gt[i];
        if (flags & ORACLE_GATE)
          gl = lower_bound * sigmoidf_ref(head_scale * (gl + dt_bias[h * K + i]));
        al[i] = expf(gl);
      }
      float b = beta[(size_t)t * H + h];
      if (flags & ORACLE_BETA_SIGMOID) b = sigmoidf_ref(b);
      for (int j = 0; j < V; ++j) pred[j] = 0.f;
      for (int i = 0; i < K; ++i) {
        float *row = S + (size_t)i * V;
        const float a = al[i], kk = kn[i];
        for (int j = 0; j < V; ++j) {
          row[j] *= a;
          pred[j] += kk * row[j];
        }
      }
      for (int j = 0; j < V; ++j) { pred[j] = (vt[j] - pred[j]) * b; acc[j] = 0.f; }
      for (int i = 0; i < K; ++i) {
        float *row = S + (size_t)i * V;
        const float kk = kn[i], qq = qn[i];
        for (int j = 0; j < V; ++j) {
          row[j] += kk * pred[j];
          acc[j] += qq * row[j];
        }
      }
      float *ot = o + ((size_t)t * H + h) * V;
      for (int j = 0; j < V; ++j) ot[j] = acc[j];
    }
    if (ht) memcpy(ht + soff, S, sizeof(float) * (size_t)K * V);
    free(S); free(qn); free(kn); free(al); free(pred); free(acc);
  }
  return bad ? -2 : 0;
}

int oracle_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
