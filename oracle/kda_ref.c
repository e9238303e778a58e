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

/*
 * Gradients of oracle_kda_varlen_f32 (the chain rule through the per-token
 * recurrence; what FlashKDAFunction.backward returns,
 * ml/training/pretrain/engine/sm120_concurrent_ffn.py:301-373).  Per
 * (sequence, head): the state at every 64-token chunk start is kept, and each
 * chunk is recomputed with all its states before its reverse steps.
 *   d_out: [T, H, V]; d_ht: [N, H, K, V] or NULL.
 *   dq, dk, dg: [T, H, K]; dv: [T, H, V]; dbeta: [T, H]; dh0: [N, H, K, V];
 *   dA_part: [N, H] and dbias_part: [N, H, K] (per-sequence sums, with the gate).
 */
int oracle_kda_varlen_bwd_f32(const float *q, const float *k, const float *v, const float *g,
                              const float *beta, const float *A_log, const float *dt_bias,
                              float lower_bound, float scale, int flags, const int32_t *cu_seqlens,
                              int n_seqs, int H, int K, int V, const float *h0, const float *d_out,
                              const float *d_ht, float *dq, float *dk, float *dv, float *dg,
                              float *dbeta, float *dh0, float *dA_part, float *dbias_part,
                              int nthreads) {
  if (K <= 0 || V <= 0 || H <= 0 || n_seqs < 0) return -1;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#else
  (void)nthreads;
#endif
  const int C = 64;
  const size_t KV = (size_t)K * V;
  const long pairs = (long)n_seqs * H;
  int bad = 0;
#pragma omp parallel for schedule(dynamic, 1)
  for (long pr = 0; pr < pairs; ++pr) {
    const int s = (int)(pr / H), h = (int)(pr % H);
    const int t0 = cu_seqlens[s], T = cu_seqlens[s + 1] - cu_seqlens[s];
    const int nch = (T + C - 1) / C;
    float *ck = (float *)malloc(sizeof(float) * KV * (size_t)(nch > 0 ? nch : 1));
    float *st = (float *)malloc(sizeof(float) * KV * (size_t)(C + 1));
    float *dS = (float *)malloc(sizeof(float) * KV);
    float *qn = (float *)malloc(sizeof(float) * (size_t)K * (T > 0 ? T : 1));
    float *kn = (float *)malloc(sizeof(float) * (size_t)K * (T > 0 ? T : 1));
    float *al = (float *)malloc(sizeof(float) * (size_t)K * (T > 0 ? T : 1));
    float *bt = (float *)malloc(sizeof(float) * (size_t)(T > 0 ? T : 1));
    float *p = (float *)malloc(sizeof(float) * (size_t)V);
    float *u = (float *)malloc(sizeof(float) * (size_t)V);
    float *du = (float *)malloc(sizeof(float) * (size_t)V);
    float *dqh = (float *)malloc(sizeof(float) * (size_t)K);
    float *dkh = (float *)malloc(sizeof(float) * (size_t)K);
    float *dal = (float *)malloc(sizeof(float) * (size_t)K);
    if (!ck || !st || !dS || !qn || !kn || !al || !bt || !p || !u || !du || !dqh || !dkh || !dal) {
#pragma omp atomic write
      bad = 1;
      free(ck); free(st); free(dS); free(qn); free(kn); free(al); free(bt); free(p); free(u); free(du);
      free(dqh); free(dkh); free(dal);
      continue;
    }
    const float head_scale = A_log ? expf(A_log[h]) : 1.0f;
    /* prepared inputs */
    for (int t = 0; t < T; ++t) {
      const size_t r = ((size_t)(t0 + t) * H + h) * K;
      float qs = scale, ks = 1.0f;
      if (flags & ORACLE_QK_L2NORM) {
        float sq = 0.f, sk = 0.f;
        for (int i = 0; i < K; ++i) { sq += q[r + i] * q[r + i]; sk += k[r + i] * k[r + i]; }
        qs = scale / fmaxf(sqrtf(sq), 1e-12f);
        ks = 1.0f / fmaxf(sqrtf(sk), 1e-12f);
      }
      for (int i = 0; i < K; ++i) {
        qn[(size_t)t * K + i] = q[r + i] * qs;
        kn[(size_t)t * K + i] = k[r + i] * ks;
        float gl = g[r + i];
        if (flags & ORACLE_GATE) gl = lower_bound * sigmoidf_ref(head_scale * (gl + dt_bias[h * K + i]));
        al[(size_t)t * K + i] = expf(gl);
      }
      float b = beta[(size_t)(t0 + t) * H + h];
      if (flags & ORACLE_BETA_SIGMOID) b = sigmoidf_ref(b);
      bt[t] = b;
    }
    /* one forward step: S (K x V) from its predecessor, p and u of the token */
#define FWD_STEP(Sin, Sout, t)                                                        \
    do {                                                                              \
      for (int j = 0; j < V; ++j) p[j] = 0.f;                                         \
      for (int i = 0; i < K; ++i) {                                                   \
        const float a_ = al[(size_t)(t) * K + i], k_ = kn[(size_t)(t) * K + i];       \
        for (int j = 0; j < V; ++j) {                                                 \
          const float x_ = (Sin)[(size_t)i * V + j] * a_;                             \
          (Sout)[(size_t)i * V + j] = x_;                                             \
          p[j] += k_ * x_;                                                            \
        }                                                                             \
      }                                                                               \
      const float *vt_ = v + ((size_t)(t0 + (t)) * H + h) * V;                        \
      for (int j = 0; j < V; ++j) u[j] = bt[t] * (vt_[j] - p[j]);                     \
      for (int i = 0; i < K; ++i) {                                                   \
        const float k_ = kn[(size_t)(t) * K + i];                                     \
        for (int j = 0; j < V; ++j) (Sout)[(size_t)i * V + j] += k_ * u[j];           \
      }                                                                               \
    } while (0)
    /* forward: chunk-start states */
    const size_t soff = ((size_t)s * H + h) * KV;
    if (h0) memcpy(st, h0 + soff, sizeof(float) * KV); else memset(st, 0, sizeof(float) * KV);
    for (int c = 0; c < nch; ++c) {
      memcpy(ck + (size_t)c * KV, st, sizeof(float) * KV);
      const int n = T - c * C < C ? T - c * C : C;
      for (int t = 0; t < n; ++t) FWD_STEP(st, st, c * C + t);
    }
    if (d_ht) memcpy(dS, d_ht + soff, sizeof(float) * KV); else memset(dS, 0, sizeof(float) * KV);
    for (int c = nch - 1; c >= 0; --c) {
      const int n = T - c * C < C ? T - c * C : C;
      memcpy(st, ck + (size_t)c * KV, sizeof(float) * KV);
      for (int t = 0; t < n; ++t) FWD_STEP(st + (size_t)t * KV, st + (size_t)(t + 1) * KV, c * C + t);
      for (int tt = n - 1; tt >= 0; --tt) {
        const int t = c * C + tt;
        const float *Sprev = st + (size_t)tt * KV, *Scur = st + (size_t)(tt + 1) * KV;
        const float *dot = d_out + ((size_t)(t0 + t) * H + h) * V;
        const float *vt = v + ((size_t)(t0 + t) * H + h) * V;
        const float b = bt[t];
        /* p and u of this token again */
        for (int j = 0; j < V; ++j) p[j] = 0.f;
        for (int i = 0; i < K; ++i)
          for (int j = 0; j < V; ++j) p[j] += kn[(size_t)t * K + i] * al[(size_t)t * K + i] * Sprev[(size_t)i * V + j];
        for (int j = 0; j < V; ++j) { u[j] = b * (vt[j] - p[j]); du[j] = 0.f; }
        for (int i = 0; i < K; ++i) {
          const float qi = qn[(size_t)t * K + i], ki = kn[(size_t)t * K + i];
          float acc = 0.f;
          for (int j = 0; j < V; ++j) {
            dS[(size_t)i * V + j] += qi * dot[j];
            acc += Scur[(size_t)i * V + j] * dot[j];
            du[j] += ki * dS[(size_t)i * V + j];
          }
          dqh[i] = acc;
        }
        float db = 0.f;
        float *dvt = dv + ((size_t)(t0 + t) * H + h) * V;
        for (int j = 0; j < V; ++j) {
          dvt[j] = b * du[j];
          db += du[j] * (vt[j] - p[j]);
        }
        for (int i = 0; i < K; ++i) {
          const float ai = al[(size_t)t * K + i], ki = kn[(size_t)t * K + i];
          float a1 = 0.f, a2 = 0.f;
          for (int j = 0; j < V; ++j) {
            const float dp = -b * du[j];
            const float sprev = Sprev[(size_t)i * V + j];
            const float dsij = dS[(size_t)i * V + j];
            a1 += dsij * u[j] + ai * sprev * dp;
            const float dst = dsij + ki * dp;
            a2 += dst * sprev;
            dS[(size_t)i * V + j] = ai * dst;
          }
          dkh[i] = a1;
          dal[i] = a2;
        }
        /* input gradients of the token */
        const size_t r = ((size_t)(t0 + t) * H + h) * K;
        if (flags & ORACLE_QK_L2NORM) {
          float sq = 0.f, sk = 0.f, yq = 0.f, yk = 0.f;
          for (int i = 0; i < K; ++i) { sq += q[r + i] * q[r + i]; sk += k[r + i] * k[r + i]; }
          const float nq = fmaxf(sqrtf(sq), 1e-12f), nk = fmaxf(sqrtf(sk), 1e-12f);
          for (int i = 0; i < K; ++i) { yq += q[r + i] / nq * dqh[i] * scale; yk += k[r + i] / nk * dkh[i]; }
          for (int i = 0; i < K; ++i) {
            dq[r + i] = (dqh[i] * scale - (sqrtf(sq) >= 1e-12f ? q[r + i] / nq * yq : 0.f)) / nq;
            dk[r + i] = (dkh[i] - (sqrtf(sk) >= 1e-12f ? k[r + i] / nk * yk : 0.f)) / nk;
          }
        } else {
          for (int i = 0; i < K; ++i) { dq[r + i] = dqh[i] * scale; dk[r + i] = dkh[i]; }
        }
        for (int i = 0; i < K; ++i) {
          float dgv = dal[i] * al[(size_t)t * K + i];
          if (flags & ORACLE_GATE) {
            const float zb = g[r + i] + dt_bias[h * K + i];
            const float sg = sigmoidf_ref(head_scale * zb);
            dgv *= lower_bound * sg * (1.f - sg) * head_scale;
            if (dbias_part) dbias_part[((size_t)s * H + h) * K + i] += dgv;
            if (dA_part) dA_part[(size_t)s * H + h] += dgv * zb;
          }
          dg[r + i] = dgv;
        }
        dbeta[(size_t)(t0 + t) * H + h] = (flags & ORACLE_BETA_SIGMOID) ? db * b * (1.f - b) : db;
      }
    }
#undef FWD_STEP
    if (dh0) memcpy(dh0 + soff, dS, sizeof(float) * KV);
    free(ck); free(st); free(dS); free(qn); free(kn); free(al); free(bt); free(p); free(u); free(du);
    free(dqh); free(dkh); free(dal);
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
