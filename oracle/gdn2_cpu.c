/*
 * C restatement of the gdn2 token recurrence -- TEST INFRASTRUCTURE ONLY.
 *
 * Used by tests/ (cross-checked against the float64 numpy oracle) and by the
 * cpu_baseline leg of bench.py (timed on the host cores).  The product library
 * (qwendopamine_amd/csrc) never links or calls it.
 *
 * Restates reference models/gdn2/gdn2.py:100-184 (torch_recurrent_gdn2) in
 * float32, the precision that function computes in (gdn2.py:132-137):
 *   q, k <- F.normalize(., eps=1e-6) (gdn2.py:139-141); q <- q * scale (143-144)
 *   per token:  S <- Diag(exp(g)) S ; r = S^T (b*k) ; u = w*v - r ;
 *               S <- S + k u^T ; o = S^T q                  (gdn2.py:156-179)
 * Layouts: q,k,g,b [B,T,H,K]; v,w,o [B,T,H,V]; states [B,H,K,V] (V fastest).
 * Sequences (b,h) are independent and are split over OpenMP threads.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>

static void normalize_scaled(const float *x, float *y, int n, float scale, int l2)
{
    float inv = 1.0f;
    if (l2) {
        double ss = 0.0;
        for (int i = 0; i < n; ++i) ss += (double)x[i] * x[i];
        double nrm = sqrt(ss);
        inv = (float)(1.0 / (nrm > 1e-6 ? nrm : 1e-6));
    }
    for (int i = 0; i < n; ++i) y[i] = x[i] * inv * scale;
}

int gdn2_cpu_recurrent_fwd_f32(const float *q, const float *k, const float *v, const float *g,
                               const float *b, const float *w, const float *h0, float *o,
                               float *ht, int B, int T, int H, int K, int V, float scale,
                               int l2norm, int nthreads)
{
    if (B < 0 || T < 0 || H <= 0 || K <= 0 || V <= 0) return -1;
    if (nthreads > 0) omp_set_num_threads(nthreads);
    int fail = 0;
#pragma omp parallel for schedule(dynamic, 1)
    for (int bh = 0; bh < B * H; ++bh) {
        const int bi = bh / H, h = bh % H;
        float *S = (float *)malloc(sizeof(float) * (size_t)K * V);
        float *qs = (float *)malloc(sizeof(float) * (size_t)K);
        float *kn = (float *)malloc(sizeof(float) * (size_t)K);
        float *ek = (float *)malloc(sizeof(float) * (size_t)K);
        float *ag = (float *)malloc(sizeof(float) * (size_t)K);
        float *u = (float *)malloc(sizeof(float) * (size_t)V);
        if (!S || !qs || !kn || !ek || !ag || !u) {
#pragma omp atomic write
            fail = 1;
        } else {
            if (h0)
                memcpy(S, h0 + (size_t)bh * K * V, sizeof(float) * (size_t)K * V);
            else
                memset(S, 0, sizeof(float) * (size_t)K * V);
            for (int t = 0; t < T; ++t) {
                const size_t rk = ((size_t)(bi * T + t) * H + h) * K;
                const size_t rv = ((size_t)(bi * T + t) * H + h) * V;
                normalize_scaled(q + rk, qs, K, scale, l2norm);
                normalize_scaled(k + rk, kn, K, 1.0f, l2norm);
                for (int d = 0; d < K; ++d) {
                    ag[d] = expf(g[rk + d]);
                    ek[d] = b[rk + d] * kn[d];
                }
                for (int c = 0; c < V; ++c) u[c] = 0.0f;
                for (int d = 0; d < K; ++d) {
                    float *row = S + (size_t)d * V;
                    const float a = ag[d], e = ek[d];
                    for (int c = 0; c < V; ++c) {
                        row[c] *= a;
                        u[c] += row[c] * e;
                    }
                }
                for (int c = 0; c < V; ++c) u[c] = w[rv + c] * v[rv + c] - u[c];
                float *orow = o + rv;
                for (int c = 0; c < V; ++c) orow[c] = 0.0f;
                for (int d = 0; d < K; ++d) {
                    float *row = S + (size_t)d * V;
                    const float kd = kn[d], qd = qs[d];
                    for (int c = 0; c < V; ++c) {
                        row[c] += kd * u[c];
                        orow[c] += row[c] * qd;
                    }
                }
            }
            if (ht) memcpy(ht + (size_t)bh * K * V, S, sizeof(float) * (size_t)K * V);
        }
        free(S); free(qs); free(kn); free(ek); free(ag); free(u);
    }
    return fail ? -2 : 0;
}

int gdn2_cpu_max_threads(void) { return omp_get_max_threads(); }
