/*
 * CPU oracle for the WKV7 recurrence, float64 -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this library, as the checker.  The product path never links it.
 *
 * forward  : restates theseus/wkv7.py:16-28 and kernels/wkv7_state.cu:20-39.
 * backward : restates the adjoint of kernels/wkv7_state.cu:49-78.
 * Layouts  : token vectors [B,T,H,N] at ((b*T+t)*H+h)*N+n (cu:25);
 *            state [B,H,N,N] at ((b*H+h)*N+i)*N+j, i = value row, j = key
 *            column (cu:21).
 * mode     : 0 = the reference's decay exp(-e^{-1/2} sigmoid(w)) (cu:27);
 *            1 = exp(w), unclamped (the GDN teacher's decay,
 *            convert_qwen2rwkv_lightning.py:384).
 * Parallel over (b,h) with OpenMP; every (b,h) is independent, so results
 * do not depend on the thread count.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#define DECAY_SCALE 0.6065306597126334 /* e^{-1/2}, cu:27 */

static inline double sigm(double x) { return 1.0 / (1.0 + exp(-x)); }

static inline double dec(int mode, double w) { return mode ? exp(w) : exp(-DECAY_SCALE * sigm(w)); }
/* d(log d)/dw */
static inline double dlogd(int mode, double w) {
    if (mode) return 1.0;
    double s = sigm(w);
    return -DECAY_SCALE * s * (1.0 - s);
}

static inline long tok(int b, int t, int h, int T, int H, int N) {
    return (((long)b * T + t) * H + h) * N;
}

void wkv7_oracle_forward(int B, int T, int H, int N, int mode, const double* r, const double* w,
                         const double* k, const double* v, const double* a, const double* b,
                         const double* s0, double* y, double* sT) {
#pragma omp parallel for schedule(dynamic)
    for (int bh = 0; bh < B * H; bh++) {
        int bb = bh / H, h = bh % H;
        double* S = (double*)malloc(sizeof(double) * N * N);
        double* d = (double*)malloc(sizeof(double) * N);
        double* sa = (double*)malloc(sizeof(double) * N);
        memcpy(S, s0 + (long)bh * N * N, sizeof(double) * N * N);
        for (int t = 0; t < T; t++) {
            long o = tok(bb, t, h, T, H, N);
            for (int j = 0; j < N; j++) d[j] = dec(mode, w[o + j]);
            for (int i = 0; i < N; i++) {           /* sa_i = sum_j S_ij a_j */
                double acc = 0.0;
                for (int j = 0; j < N; j++) acc += S[i * N + j] * a[o + j];
                sa[i] = acc;
            }
            for (int i = 0; i < N; i++) {
                double acc = 0.0;
                for (int j = 0; j < N; j++) {
                    double s = S[i * N + j] * d[j] + sa[i] * b[o + j] + v[o + i] * k[o + j];
                    S[i * N + j] = s;
                    acc += s * r[o + j];
                }
                y[o + i] = acc;
            }
        }
        memcpy(sT + (long)bh * N * N, S, sizeof(double) * N * N);
        free(S); free(d); free(sa);
    }
}

void wkv7_oracle_backward(int B, int T, int H, int N, int mode, const double* r, const double* w,
                          const double* k, const double* v, const double* a, const double* b,
                          const double* s0, const double* dy, const double* dsT,
                          double* dr, double* dw, double* dk, double* dv, double* da,
                          double* db, double* ds0) {
#pragma omp parallel for schedule(dynamic)
    for (int bh = 0; bh < B * H; bh++) {
        int bb = bh / H, h = bh % H;
        long NN = (long)N * N;
        /* full per-(b,h) history S_0..S_T, recomputed in float64 */
        double* hist = (double*)malloc(sizeof(double) * NN * (T + 1));
        double* G = (double*)malloc(sizeof(double) * NN);
        double* sa = (double*)malloc(sizeof(double) * N);
        double* q = (double*)malloc(sizeof(double) * N);
        double* d = (double*)malloc(sizeof(double) * N);
        memcpy(hist, s0 + (long)bh * NN, sizeof(double) * NN);
        for (int t = 0; t < T; t++) {
            long o = tok(bb, t, h, T, H, N);
            const double* Sp = hist + NN * t;
            double* Sn = hist + NN * (t + 1);
            for (int j = 0; j < N; j++) d[j] = dec(mode, w[o + j]);
            for (int i = 0; i < N; i++) {
                double acc = 0.0;
                for (int j = 0; j < N; j++) acc += Sp[i * N + j] * a[o + j];
                sa[i] = acc;
            }
            for (int i = 0; i < N; i++)
                for (int j = 0; j < N; j++)
                    Sn[i * N + j] = Sp[i * N + j] * d[j] + sa[i] * b[o + j] + v[o + i] * k[o + j];
        }
        memcpy(G, dsT + (long)bh * NN, sizeof(double) * NN);     /* cu:50 */
        for (int t = T - 1; t >= 0; t--) {
            long o = tok(bb, t, h, T, H, N);
            const double* Sp = hist + NN * t;
            const double* Sn = hist + NN * (t + 1);
            for (int i = 0; i < N; i++) {                     /* cu:61-65 */
                double acc = 0.0, accq = 0.0;
                for (int j = 0; j < N; j++) acc += Sp[i * N + j] * a[o + j];
                sa[i] = acc;
                for (int j = 0; j < N; j++) {
                    G[i * N + j] += dy[o + i] * r[o + j];
                    accq += G[i * N + j] * b[o + j];
                }
                q[i] = accq;
            }
            for (int j = 0; j < N; j++) {                     /* cu:68-72 */
                double dj = dec(mode, w[o + j]);
                double gr = 0, gw = 0, gk = 0, gb = 0, ga = 0;
                for (int i = 0; i < N; i++) {
                    double g = G[i * N + j];
                    gr += dy[o + i] * Sn[i * N + j];
                    gw += g * Sp[i * N + j];
                    gk += g * v[o + i];
                    gb += g * sa[i];
                    ga += q[i] * Sp[i * N + j];
                }
                dr[o + j] = gr;
                dw[o + j] = gw * dj * dlogd(mode, w[o + j]);
                dk[o + j] = gk;
                db[o + j] = gb;
                da[o + j] = ga;
            }
            for (int i = 0; i < N; i++) {                     /* cu:73,76 */
                double acc = 0.0;
                for (int j = 0; j < N; j++) acc += G[i * N + j] * k[o + j];
                dv[o + i] = acc;
            }
            for (int j = 0; j < N; j++) d[j] = dec(mode, w[o + j]);
            for (int i = 0; i < N; i++)                       /* cu:74 */
                for (int j = 0; j < N; j++)
                    G[i * N + j] = G[i * N + j] * d[j] + q[i] * a[o + j];
        }
        memcpy(ds0 + (long)bh * NN, G, sizeof(double) * NN); /* cu:78 */
        free(hist); free(G); free(sa); free(q); free(d);
    }
}
