/*
 * aic_oracle.c -- CPU restatement of the AutonomousAICore TransformerLM training step.
 *
 * TEST INFRASTRUCTURE ONLY (see aic_oracle.h).  Built with -ffp-contract=off so that the
 * only fused multiply-adds are the explicit AVX2 ones of the GEMM microkernel, as in the
 * reference (src/ops/cpu_gemm.cpp:20-62).  Reductions accumulate in double where the
 * reference does (src/ops/cpu_ops.cpp:152-269, src/loss/cross_entropy.cpp:214-222,
 * src/optim/clip_grad.cpp:25-32).
 */
#define _GNU_SOURCE
#include "aic_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <unistd.h>

static int g_threads = 0;

void orc_set_threads(int n) { g_threads = n; }

int orc_get_threads(void) {
    if (g_threads > 0) return g_threads;
    long hw = sysconf(_SC_NPROCESSORS_ONLN);
    int n = hw <= 0 ? 4 : (int)hw;
    if (n > 24) n = 24;  /* src/ops/cpu_gemm.cpp:143-146 */
    return n;
}

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

static void* xcalloc(size_t n, size_t sz) {
    void* p = calloc(n ? n : 1, sz);
    if (!p) abort();
    return p;
}

/* ======================================================================================
 * GEMM (src/ops/cpu_gemm.cpp)
 * ====================================================================================== */

/* 4x16 AVX2+FMA microkernel, accumulating into C (src/ops/cpu_gemm.cpp:20-62). */
static void mk_4x16(int64_t kl, const float* a, int64_t lda, const float* b, int64_t ldb, float* c, int64_t ldc) {
    __m256 c00 = _mm256_loadu_ps(c + 0 * ldc + 0), c01 = _mm256_loadu_ps(c + 0 * ldc + 8);
    __m256 c10 = _mm256_loadu_ps(c + 1 * ldc + 0), c11 = _mm256_loadu_ps(c + 1 * ldc + 8);
    __m256 c20 = _mm256_loadu_ps(c + 2 * ldc + 0), c21 = _mm256_loadu_ps(c + 2 * ldc + 8);
    __m256 c30 = _mm256_loadu_ps(c + 3 * ldc + 0), c31 = _mm256_loadu_ps(c + 3 * ldc + 8);
    for (int64_t p = 0; p < kl; ++p) {
        __m256 b0 = _mm256_loadu_ps(b + p * ldb), b1 = _mm256_loadu_ps(b + p * ldb + 8);
        __m256 a0 = _mm256_set1_ps(a[0 * lda + p]);
        __m256 a1 = _mm256_set1_ps(a[1 * lda + p]);
        __m256 a2 = _mm256_set1_ps(a[2 * lda + p]);
        __m256 a3 = _mm256_set1_ps(a[3 * lda + p]);
        c00 = _mm256_fmadd_ps(a0, b0, c00); c01 = _mm256_fmadd_ps(a0, b1, c01);
        c10 = _mm256_fmadd_ps(a1, b0, c10); c11 = _mm256_fmadd_ps(a1, b1, c11);
        c20 = _mm256_fmadd_ps(a2, b0, c20); c21 = _mm256_fmadd_ps(a2, b1, c21);
        c30 = _mm256_fmadd_ps(a3, b0, c30); c31 = _mm256_fmadd_ps(a3, b1, c31);
    }
    _mm256_storeu_ps(c + 0 * ldc, c00); _mm256_storeu_ps(c + 0 * ldc + 8, c01);
    _mm256_storeu_ps(c + 1 * ldc, c10); _mm256_storeu_ps(c + 1 * ldc + 8, c11);
    _mm256_storeu_ps(c + 2 * ldc, c20); _mm256_storeu_ps(c + 2 * ldc + 8, c21);
    _mm256_storeu_ps(c + 3 * ldc, c30); _mm256_storeu_ps(c + 3 * ldc + 8, c31);
}

/* 64x64 K/N tiling over rows [m0, m1) (src/ops/cpu_gemm.cpp:65-115). */
static void block_tiled(int64_t m0, int64_t m1, int64_t N, int64_t K, const float* A, const float* B, float* C) {
    const int64_t TN = 64, TK = 64;
    for (int64_t kb = 0; kb < K; kb += TK) {
        int64_t kl = (kb + TK <= K) ? TK : (K - kb);
        for (int64_t nb = 0; nb < N; nb += TN) {
            int64_t nl = (nb + TN <= N) ? TN : (N - nb);
            int64_t m = m0;
            for (; m + 4 <= m1; m += 4) {
                int64_t n = nb;
                for (; n + 16 <= nb + nl; n += 16)
                    mk_4x16(kl, A + m * K + kb, K, B + kb * N + n, N, C + m * N + n, N);
                for (; n < nb + nl; ++n) {
                    for (int64_t sm = 0; sm < 4; ++sm) {
                        float sum = 0.0f;
                        for (int64_t p = 0; p < kl; ++p) sum += A[(m + sm) * K + kb + p] * B[(kb + p) * N + n];
                        C[(m + sm) * N + n] += sum;
                    }
                }
            }
            for (; m < m1; ++m) {
                for (int64_t n = nb; n < nb + nl; ++n) {
                    float sum = 0.0f;
                    for (int64_t p = 0; p < kl; ++p) sum += A[m * K + kb + p] * B[(kb + p) * N + n];
                    C[m * N + n] += sum;
                }
            }
        }
    }
}

typedef struct {
    int64_t m0, m1, N, K;
    const float *A, *B;
    float* C;
} gemm_job;

static void* gemm_worker(void* arg) {
    gemm_job* j = (gemm_job*)arg;
    block_tiled(j->m0, j->m1, j->N, j->K, j->A, j->B, j->C);
    return NULL;
}

/* gemm_2d (src/ops/cpu_gemm.cpp:119-177): C zero-initialised, then a row split over
 * min(hw, 24) threads, single-threaded for small problems. */
void orc_gemm(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K) {
    memset(C, 0, sizeof(float) * (size_t)(M * N));
    if (M == 0 || N == 0 || K == 0) return;
    int nt = orc_get_threads();
    int64_t work = M * N * K;
    if (M < (int64_t)nt * 4 || work < 64 * 64 * 64) nt = 1;
    if (nt == 1) {
        block_tiled(0, M, N, K, A, B, C);
        return;
    }
    int64_t rpt = (M + nt - 1) / nt;
    rpt = ((rpt + 3) / 4) * 4;
    pthread_t th[64];
    gemm_job jobs[64];
    int launched = 0;
    for (int t = 0; t < nt; ++t) {
        int64_t m0 = t * rpt;
        if (m0 >= M) break;
        int64_t m1 = (m0 + rpt <= M) ? m0 + rpt : M;
        jobs[t] = (gemm_job){m0, m1, N, K, A, B, C};
        pthread_create(&th[t], NULL, gemm_worker, &jobs[t]);
        ++launched;
    }
    for (int t = 0; t < launched; ++t) pthread_join(th[t], NULL);
}

static void transpose(const float* src, float* dst, int64_t rows, int64_t cols) {
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < cols; ++c) dst[c * rows + r] = src[r * cols + c];
}

/* Linear forward: matmul(x, W^T) with W^T made contiguous, one gemm_2d per batch
 * (include/nn/linear.hpp:31-41, src/ops/cpu_gemm.cpp:180-254). */
void orc_linear_fwd(const float* x, const float* W, float* y, int64_t B, int64_t S, int64_t in, int64_t out) {
    float* Wt = (float*)xcalloc((size_t)(in * out), sizeof(float));
    transpose(W, Wt, out, in);
    for (int64_t b = 0; b < B; ++b) orc_gemm(x + b * S * in, Wt, y + b * S * out, S, out, in);
    free(Wt);
}

/* MatMulBackward of y = x . W^T (src/autograd/functions.cpp:254-273):
 *   grad_a = matmul(g, W)            -> dx_b = dy_b . W            (per batch)
 *   grad_b = matmul(x^T, g)          -> P_b = x_b^T . dy_b  [in,out]
 *   reduce_gradient_for_broadcast    -> sum over b in double      (src/ops/cpu_ops.cpp:195-262)
 *   TransposeBackward                -> dW = (sum_b P_b)^T [out,in]
 * dW is accumulated (+=) into the caller's buffer, as AccumulateGrad adds to an existing
 * gradient (src/autograd/node.cpp:31-46). */
void orc_linear_bwd(const float* x, const float* W, const float* dy, float* dx, float* dW,
                    int64_t B, int64_t S, int64_t in, int64_t out) {
    if (dx) {
        for (int64_t b = 0; b < B; ++b) orc_gemm(dy + b * S * out, W, dx + b * S * in, S, in, out);
    }
    if (dW) {
        float* xt = (float*)xcalloc((size_t)(in * S), sizeof(float));
        float* Pb = (float*)xcalloc((size_t)(in * out), sizeof(float));
        double* acc = (double*)xcalloc((size_t)(in * out), sizeof(double));
        for (int64_t b = 0; b < B; ++b) {
            transpose(x + b * S * in, xt, S, in);
            orc_gemm(xt, dy + b * S * out, Pb, in, out, S);
            for (int64_t i = 0; i < in * out; ++i) acc[i] += (double)Pb[i];
        }
        for (int64_t i = 0; i < in; ++i)
            for (int64_t o = 0; o < out; ++o) dW[o * in + i] += (float)acc[i * out + o];
        free(acc);
        free(Pb);
        free(xt);
    }
}

/* ======================================================================================
 * RMSNorm (include/nn/rms_norm.hpp:18-34)
 *   x2 = x*x; mean(x2,-1) in double -> float; rms = sqrt(mean + eps); y = (x / rms) * w
 * ====================================================================================== */
void orc_rmsnorm_fwd(const float* x, const float* w, float* y, float* rms, int64_t rows, int64_t d, float eps) {
    for (int64_t r = 0; r < rows; ++r) {
        const float* xr = x + r * d;
        double acc = 0.0;
        for (int64_t j = 0; j < d; ++j) {
            float sq = xr[j] * xr[j];
            acc += (double)sq;
        }
        float mean = (float)(acc / (double)d);
        float rr = sqrtf(mean + eps);
        if (rms) rms[r] = rr;
        for (int64_t j = 0; j < d; ++j) {
            float n = xr[j] / rr;
            y[r * d + j] = n * w[j];
        }
    }
}

/* Closed-form gradient of the graph above (MulBackward, DivBackward, SqrtBackward,
 * MeanBackward, src/autograd/functions.cpp:60-78,150-200):
 *   dn = dy*w;  dx_j = dn_j/rms - x_j * sum_i(dn_i x_i) / (d rms^3);  dw_j += sum_rows dy_j x_j/rms
 * dx is written (not accumulated); dw is accumulated. */
void orc_rmsnorm_bwd(const float* dy, const float* x, const float* w, const float* rms,
                     float* dx, float* dw, int64_t rows, int64_t d) {
    double* dwacc = dw ? (double*)xcalloc((size_t)d, sizeof(double)) : NULL;
    for (int64_t r = 0; r < rows; ++r) {
        const float* xr = x + r * d;
        const float* gr = dy + r * d;
        float rr = rms[r];
        double dot = 0.0;
        for (int64_t j = 0; j < d; ++j) dot += (double)(gr[j] * w[j]) * (double)xr[j];
        float coef = (float)(dot / ((double)d * (double)rr * (double)rr * (double)rr));
        if (dx)
            for (int64_t j = 0; j < d; ++j) dx[r * d + j] = (gr[j] * w[j]) / rr - xr[j] * coef;
        if (dwacc)
            for (int64_t j = 0; j < d; ++j) dwacc[j] += (double)(gr[j] * (xr[j] / rr));
    }
    if (dw) {
        for (int64_t j = 0; j < d; ++j) dw[j] += (float)dwacc[j];
        free(dwacc);
    }
}

/* ======================================================================================
 * RoPE (include/nn/rope.hpp)
 * ====================================================================================== */
void orc_rope_tables(float* cos_t, float* sin_t, int64_t max_seq, int64_t hd, float base) {
    int64_t half = hd / 2;
    float* freqs = (float*)xcalloc((size_t)half, sizeof(float));
    for (int64_t i = 0; i < half; ++i) {
        float exponent = (float)(2 * i) / (float)hd;
        freqs[i] = 1.0f / powf(base, exponent);
    }
    for (int64_t pos = 0; pos < max_seq; ++pos)
        for (int64_t i = 0; i < half; ++i) {
            float angle = (float)pos * freqs[i];
            cos_t[pos * half + i] = cosf(angle);
            sin_t[pos * half + i] = sinf(angle);
        }
    free(freqs);
}

/* x1' = x1*c - x2*s ; x2' = x1*s + x2*c (include/nn/rope.hpp:97-99). */
void orc_rope_fwd(float* x, const float* cos_t, const float* sin_t, int64_t B, int64_t S, int64_t H,
                  int64_t hd, int64_t start_pos) {
    int64_t half = hd / 2;
    for (int64_t b = 0; b < B; ++b)
        for (int64_t s = 0; s < S; ++s)
            for (int64_t h = 0; h < H; ++h) {
                float* row = x + ((b * S + s) * H + h) * hd;
                const float* c = cos_t + (start_pos + s) * half;
                const float* sn = sin_t + (start_pos + s) * half;
                for (int64_t i = 0; i < half; ++i) {
                    float x1 = row[i], x2 = row[i + half];
                    float a = x1 * c[i], bb = x2 * sn[i];
                    float r1 = a - bb;
                    float e = x1 * sn[i], f = x2 * c[i];
                    float r2 = e + f;
                    row[i] = r1;
                    row[i + half] = r2;
                }
            }
}

/* dx1 = g1*c + g2*s ; dx2 = g2*c - g1*s (include/nn/rope.hpp:23-39). */
void orc_rope_bwd(float* g, const float* cos_t, const float* sin_t, int64_t B, int64_t S, int64_t H,
                  int64_t hd, int64_t start_pos) {
    int64_t half = hd / 2;
    for (int64_t b = 0; b < B; ++b)
        for (int64_t s = 0; s < S; ++s)
            for (int64_t h = 0; h < H; ++h) {
                float* row = g + ((b * S + s) * H + h) * hd;
                const float* c = cos_t + (start_pos + s) * half;
                const float* sn = sin_t + (start_pos + s) * half;
                for (int64_t i = 0; i < half; ++i) {
                    float g1 = row[i], g2 = row[i + half];
                    float a = g1 * c[i], bb = g2 * sn[i];
                    float d1 = a + bb;
                    float e = g2 * c[i], f = g1 * sn[i];
                    float d2 = e - f;
                    row[i] = d1;
                    row[i + half] = d2;
                }
            }
}

/* ======================================================================================
 * Attention core (include/nn/attention.hpp:84-119), per (b, h) head slice:
 *   scores = gemm(q [S,hd], k^T [hd,S]); scores *= 1/sqrt(hd); scores += mask(-1e9, j > i);
 *   softmax: m = rowmax; e = exp(s - m); sum in double -> float; P = e / sum;  o = gemm(P, v)
 * ====================================================================================== */
static void gather_head(const float* x, float* dst, int64_t b, int64_t h, int64_t S, int64_t H, int64_t hd) {
    for (int64_t s = 0; s < S; ++s) memcpy(dst + s * hd, x + ((b * S + s) * H + h) * hd, sizeof(float) * (size_t)hd);
}
static void scatter_head(float* x, const float* src, int64_t b, int64_t h, int64_t S, int64_t H, int64_t hd) {
    for (int64_t s = 0; s < S; ++s) memcpy(x + ((b * S + s) * H + h) * hd, src + s * hd, sizeof(float) * (size_t)hd);
}

void orc_attention_fwd(const float* q, const float* k, const float* v, float* o, float* E, float* rowsum,
                       int64_t B, int64_t S, int64_t H, int64_t hd, int causal) {
    float scale = 1.0f / sqrtf((float)hd);
    float* qh = (float*)xcalloc((size_t)(S * hd), sizeof(float));
    float* kh = (float*)xcalloc((size_t)(S * hd), sizeof(float));
    float* kt = (float*)xcalloc((size_t)(S * hd), sizeof(float));
    float* vh = (float*)xcalloc((size_t)(S * hd), sizeof(float));
    float* oh = (float*)xcalloc((size_t)(S * hd), sizeof(float));
    float* sc = (float*)xcalloc((size_t)(S * S), sizeof(float));
    float* P = (float*)xcalloc((size_t)(S * S), sizeof(float));
    for (int64_t b = 0; b < B; ++b)
        for (int64_t h = 0; h < H; ++h) {
            gather_head(q, qh, b, h, S, H, hd);
            gather_head(k, kh, b, h, S, H, hd);
            gather_head(v, vh, b, h, S, H, hd);
            transpose(kh, kt, S, hd);
            orc_gemm(qh, kt, sc, S, S, hd);
            float* Ebh = E ? E + (b * H + h) * S * S : NULL;
            for (int64_t i = 0; i < S; ++i) {
                float* row = sc + i * S;
                for (int64_t j = 0; j < S; ++j) {
                    row[j] = row[j] * scale;
                    if (causal && S > 1 && j > i) row[j] = row[j] + (-1e9f);
                }
                float mx = row[0];
                for (int64_t j = 1; j < S; ++j)
                    if (row[j] > mx) mx = row[j];
                double acc = 0.0;
                for (int64_t j = 0; j < S; ++j) {
                    float e = expf(row[j] - mx);
                    row[j] = e;
                    acc += (double)e;
                }
                float sm = (float)acc;
                if (rowsum) rowsum[(b * H + h) * S + i] = sm;
                for (int64_t j = 0; j < S; ++j) {
                    if (Ebh) Ebh[i * S + j] = row[j];
                    P[i * S + j] = row[j] / sm;
                }
            }
            orc_gemm(P, vh, oh, S, hd, S);
            scatter_head(o, oh, b, h, S, H, hd);
        }
    free(qh); free(kh); free(kt); free(vh); free(oh); free(sc); free(P);
}

/* Flash attention's CPU forward: per query row, key blocks of 32 with a running max m, sum l
 * and accumulator rescaled by exp(m_old - m_new); masked scores are -inf and skipped. */
void orc_flash_fwd(const float* q, const float* k, const float* v, float* o, float* lse, int64_t BH, int64_t Sq,
                   int64_t Sk, int64_t D, int causal, float scale) {
    const int64_t Bc = 32;
    float* acc = (float*)xcalloc((size_t)D, sizeof(float));
    float sb[32];
    for (int64_t bh = 0; bh < BH; ++bh) {
        const float* qb = q + bh * Sq * D;
        const float* kb = k + bh * Sk * D;
        const float* vb = v + bh * Sk * D;
        for (int64_t r = 0; r < Sq; ++r) {
            const float* qr = qb + r * D;
            float m = -INFINITY, l = 0.0f;
            memset(acc, 0, sizeof(float) * (size_t)D);
            for (int64_t j0 = 0; j0 < Sk; j0 += Bc) {
                if (causal && j0 > r) break;
                const int64_t n = (j0 + Bc < Sk ? j0 + Bc : Sk) - j0;
                float bm = -INFINITY;
                for (int64_t c = 0; c < n; ++c) {
                    if (causal && j0 + c > r) {
                        sb[c] = -INFINITY;
                        continue;
                    }
                    const float* kc = kb + (j0 + c) * D;
                    float dot = 0.0f;
                    for (int64_t d = 0; d < D; ++d) dot += qr[d] * kc[d];
                    dot *= scale;
                    sb[c] = dot;
                    if (dot > bm) bm = dot;
                }
                if (bm == -INFINITY) continue;
                const float mn = m > bm ? m : bm;
                const float alpha = (m == -INFINITY) ? 0.0f : expf(m - mn);
                for (int64_t d = 0; d < D; ++d) acc[d] *= alpha;
                float bl = 0.0f;
                for (int64_t c = 0; c < n; ++c) {
                    if (!(sb[c] > -1e30f)) continue;
                    const float p = expf(sb[c] - mn);
                    bl += p;
                    const float* vc = vb + (j0 + c) * D;
                    for (int64_t d = 0; d < D; ++d) acc[d] += p * vc[d];
                }
                l = l * alpha + bl;
                m = mn;
            }
            float* orow = o + (bh * Sq + r) * D;
            if (l > 0.0f) {
                const float inv = 1.0f / l;
                for (int64_t d = 0; d < D; ++d) orow[d] = acc[d] * inv;
                lse[bh * Sq + r] = m + logf(l);
            } else {
                memset(orow, 0, sizeof(float) * (size_t)D);
                lse[bh * Sq + r] = 0.0f;
            }
        }
    }
    free(acc);
}

/* Flash attention's CPU backward: D_r = dO_r . O_r; for each visible (r, c): p = exp(s - L_r),
 * ds = p (dO_r . V_c - D_r) scale, dQ_r += ds K_c, dK_c += ds Q_r, dV_c += p dO_r. */
void orc_flash_bwd(const float* q, const float* k, const float* v, const float* o, const float* dout,
                   const float* lse, float* dq, float* dk, float* dv, int64_t BH, int64_t Sq, int64_t Sk, int64_t D,
                   int causal, float scale) {
    for (int64_t bh = 0; bh < BH; ++bh) {
        const float* qb = q + bh * Sq * D;
        const float* kb = k + bh * Sk * D;
        const float* vb = v + bh * Sk * D;
        const float* ob = o + bh * Sq * D;
        const float* gb = dout + bh * Sq * D;
        float* dqb = dq + bh * Sq * D;
        float* dkb = dk + bh * Sk * D;
        float* dvb = dv + bh * Sk * D;
        for (int64_t r = 0; r < Sq; ++r) {
            const float* qr = qb + r * D;
            const float* gr = gb + r * D;
            float Dr = 0.0f;
            for (int64_t d = 0; d < D; ++d) Dr += gr[d] * ob[r * D + d];
            const float L = lse[bh * Sq + r];
            const int64_t cmax = causal ? (r + 1 < Sk ? r + 1 : Sk) : Sk;
            for (int64_t c = 0; c < cmax; ++c) {
                const float* kc = kb + c * D;
                const float* vc = vb + c * D;
                float s = 0.0f, dp = 0.0f;
                for (int64_t d = 0; d < D; ++d) s += qr[d] * kc[d];
                s *= scale;
                const float p = expf(s - L);
                for (int64_t d = 0; d < D; ++d) dp += gr[d] * vc[d];
                const float ds = p * (dp - Dr) * scale;
                for (int64_t d = 0; d < D; ++d) {
                    dqb[r * D + d] += ds * kc[d];
                    dkb[c * D + d] += ds * qr[d];
                    dvb[c * D + d] += p * gr[d];
                }
            }
        }
    }
}

/* Backward of the graph above.  For out = e / s (DivBackward then SumBackward then ExpBackward):
 *   t_j = g_j / s ;  c = sum_k(-g_k e_k / (s*s)) in double ;  dscore_j = (t_j + c) * e_j
 * then *scale, and the two MatMulBackwards. */
void orc_attention_bwd(const float* q, const float* k, const float* v, const float* E, const float* rowsum,
                       const float* dout, float* dq, float* dk, float* dv, int64_t B, int64_t S, int64_t H,
                       int64_t hd) {
    float scale = 1.0f / sqrtf((float)hd);
    size_t sh = (size_t)(S * hd), ss = (size_t)(S * S);
    float* qh = (float*)xcalloc(sh, sizeof(float));
    float* qt = (float*)xcalloc(sh, sizeof(float));
    float* kh = (float*)xcalloc(sh, sizeof(float));
    float* vh = (float*)xcalloc(sh, sizeof(float));
    float* vt = (float*)xcalloc(sh, sizeof(float));
    float* gh = (float*)xcalloc(sh, sizeof(float));
    float* tmp = (float*)xcalloc(sh, sizeof(float));
    float* P = (float*)xcalloc(ss, sizeof(float));
    float* Pt = (float*)xcalloc(ss, sizeof(float));
    float* dP = (float*)xcalloc(ss, sizeof(float));
    for (int64_t b = 0; b < B; ++b)
        for (int64_t h = 0; h < H; ++h) {
            const float* Ebh = E + (b * H + h) * S * S;
            const float* sbh = rowsum + (b * H + h) * S;
            gather_head(q, qh, b, h, S, H, hd);
            gather_head(k, kh, b, h, S, H, hd);
            gather_head(v, vh, b, h, S, H, hd);
            gather_head(dout, gh, b, h, S, H, hd);
            for (int64_t i = 0; i < S; ++i)
                for (int64_t j = 0; j < S; ++j) P[i * S + j] = Ebh[i * S + j] / sbh[i];
            /* context = matmul(P, v): dP = g . v^T ; dv = P^T . g */
            transpose(vh, vt, S, hd);
            orc_gemm(gh, vt, dP, S, S, hd);
            transpose(P, Pt, S, S);
            orc_gemm(Pt, gh, tmp, S, hd, S);
            scatter_head(dv, tmp, b, h, S, H, hd);
            /* softmax backward */
            for (int64_t i = 0; i < S; ++i) {
                float s = sbh[i];
                const float* e = Ebh + i * S;
                float* g = dP + i * S;
                double acc = 0.0;
                for (int64_t j = 0; j < S; ++j) {
                    float t = (-g[j]) * e[j];
                    acc += (double)(t / (s * s));
                }
                float c = (float)acc;
                for (int64_t j = 0; j < S; ++j) {
                    float t = g[j] / s;
                    g[j] = ((t + c) * e[j]) * scale;
                }
            }
            /* scores = matmul(q, k^T): dq = dS . k ; d(k^T) = q^T . dS ; dk = transpose */
            orc_gemm(dP, kh, tmp, S, hd, S);
            scatter_head(dq, tmp, b, h, S, H, hd);
            transpose(qh, qt, S, hd);
            float* dkt = (float*)xcalloc(sh, sizeof(float));
            orc_gemm(qt, dP, dkt, hd, S, S);
            transpose(dkt, tmp, hd, S);
            free(dkt);
            scatter_head(dk, tmp, b, h, S, H, hd);
        }
    free(qh); free(qt); free(kh); free(vh); free(vt); free(gh); free(tmp); free(P); free(Pt); free(dP);
}

/* ======================================================================================
 * SwiGLU activation
 * ====================================================================================== */
void orc_swiglu_fwd(const float* g, const float* u, float* h, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        float x = g[i];
        float a = x / (1.0f + expf(-x)); /* silu, src/ops/cpu_ops.cpp:143-146 */
        h[i] = a * u[i];
    }
}

void orc_swiglu_bwd(const float* g, const float* u, const float* dh, float* dg, float* du, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        float x = g[i];
        float a = x / (1.0f + expf(-x));
        float s = 1.0f / (1.0f + expf(-x)); /* sigmoid, src/ops/cpu_ops.cpp:139-141 */
        float dsilu = s * (1.0f + x * (1.0f - s));
        du[i] = dh[i] * a;
        dg[i] = (dh[i] * u[i]) * dsilu;
    }
}

/* ======================================================================================
 * Cross-entropy (src/loss/cross_entropy.cpp)
 * ====================================================================================== */
float orc_ce_fwd(const float* logits, const int64_t* targets, int64_t N, int64_t C, int64_t ignore_index,
                 float* losses, float* lse_out, int64_t* valid_count) {
    int64_t valid = 0;
    double total = 0.0; /* sum(sample_losses) in double, src/ops/cpu_ops.cpp:152-162 */
    for (int64_t i = 0; i < N; ++i) {
        const float* z = logits + i * C;
        float mx = z[0];
        for (int64_t j = 1; j < C; ++j)
            if (z[j] > mx) mx = z[j];
        double se = 0.0;
        for (int64_t j = 0; j < C; ++j) se += exp((double)(z[j] - mx));
        float lse = (float)((double)mx + log(se > 1e-12 ? se : 1e-12));
        if (lse_out) lse_out[i] = lse;
        float li = 0.0f;
        int64_t t = targets[i];
        if (t != ignore_index) {
            li = lse - z[t];
            ++valid;
        }
        if (losses) losses[i] = li;
        total += (double)li;
    }
    if (valid_count) *valid_count = valid;
    if (valid == 0) return 0.0f;
    float tot = (float)total;
    return tot / (float)valid;
}

void orc_ce_bwd(const float* logits, const int64_t* targets, const float* lse, int64_t N, int64_t C,
                int64_t ignore_index, int64_t valid_count, float g, float* dlogits) {
    float scale = valid_count > 0 ? g / (float)valid_count : 0.0f;
    for (int64_t i = 0; i < N; ++i) {
        float* gz = dlogits + i * C;
        int64_t t = targets[i];
        if (t == ignore_index) {
            memset(gz, 0, sizeof(float) * (size_t)C);
            continue;
        }
        const float* z = logits + i * C;
        for (int64_t j = 0; j < C; ++j) {
            float prob = expf(z[j] - lse[i]);
            float ind = (j == t) ? 1.0f : 0.0f;
            gz[j] = (prob - ind) * scale;
        }
    }
}

/* CrossEntropyBackward's row scale for the three reductions (src/loss/cross_entropy.cpp:86-105):
 * "mean" g / valid_count (0 when no row is valid), "sum" g, "none" g[i] (1 without g). */
void orc_ce_bwd_reduction(const float* logits, const int64_t* targets, const float* lse, int64_t N, int64_t C,
                          int64_t ignore_index, int reduction, int64_t valid_count, const float* g, float* dlogits) {
    const float g_scalar = g ? g[0] : 1.0f;
    for (int64_t i = 0; i < N; ++i) {
        float* gz = dlogits + i * C;
        int64_t t = targets[i];
        if (t == ignore_index) {
            memset(gz, 0, sizeof(float) * (size_t)C);
            continue;
        }
        float scale;
        if (reduction == ORC_CE_MEAN) scale = valid_count > 0 ? g_scalar / (float)valid_count : 0.0f;
        else if (reduction == ORC_CE_SUM) scale = g_scalar;
        else scale = g ? g[i] : 1.0f;
        const float* z = logits + i * C;
        for (int64_t j = 0; j < C; ++j) {
            float prob = expf(z[j] - lse[i]);
            float ind = (j == t) ? 1.0f : 0.0f;
            gz[j] = (prob - ind) * scale;
        }
    }
}

float orc_ce_fwd_soft(const float* logits, const float* y, int64_t N, int64_t C, float* losses, float* lse_out) {
    double total = 0.0;
    for (int64_t i = 0; i < N; ++i) {
        const float* z = logits + i * C;
        const float* yr = y + i * C;
        float mx = z[0];
        for (int64_t j = 1; j < C; ++j)
            if (z[j] > mx) mx = z[j];
        double se = 0.0;
        for (int64_t j = 0; j < C; ++j) se += exp((double)(z[j] - mx));
        float lse = (float)((double)mx + log(se > 1e-12 ? se : 1e-12));
        if (lse_out) lse_out[i] = lse;
        float dot = 0.0f;
        for (int64_t j = 0; j < C; ++j) dot += yr[j] * z[j];
        float li = lse - dot;
        if (losses) losses[i] = li;
        total += (double)li;
    }
    return N > 0 ? (float)total / (float)N : 0.0f;
}

void orc_ce_bwd_soft(const float* logits, const float* y, const float* lse, int64_t N, int64_t C, const float* g,
                     int per_row, float divisor, float* dlogits) {
    for (int64_t i = 0; i < N; ++i) {
        float scale;
        if (per_row) scale = g ? g[i] : 1.0f;
        else scale = divisor > 0.0f ? (g ? g[0] : 1.0f) / divisor : 0.0f;
        const float* z = logits + i * C;
        const float* yr = y + i * C;
        float* gz = dlogits + i * C;
        for (int64_t j = 0; j < C; ++j) gz[j] = (expf(z[j] - lse[i]) - yr[j]) * scale;
    }
}

/* ======================================================================================
 * Embedding
 * ====================================================================================== */
void orc_embedding_fwd(const int64_t* ids, const float* W, float* out, int64_t N, int64_t D, int64_t V) {
    for (int64_t i = 0; i < N; ++i) {
        int64_t t = ids[i];
        if (t >= 0 && t < V) memcpy(out + i * D, W + t * D, sizeof(float) * (size_t)D);
        else memset(out + i * D, 0, sizeof(float) * (size_t)D);
    }
}

/* Scatter-add in token order; accumulates into dW. */
void orc_embedding_bwd(const int64_t* ids, const float* dout, float* dW, int64_t N, int64_t D, int64_t V) {
    for (int64_t i = 0; i < N; ++i) {
        int64_t t = ids[i];
        if (t < 0 || t >= V) continue;
        float* row = dW + t * D;
        const float* g = dout + i * D;
        for (int64_t d = 0; d < D; ++d) row[d] += g[d];
    }
}

/* ======================================================================================
 * Optimizer tail
 * ====================================================================================== */
void orc_adamw(float* p, const float* g, float* m, float* v, int64_t n, float lr, float beta1, float beta2,
               float eps, float wd, int64_t step) {
    float bc1 = 1.0f - powf(beta1, (float)step);
    float bc2 = 1.0f - powf(beta2, (float)step);
    for (int64_t i = 0; i < n; ++i) {
        float grad = g[i];
        float param = p[i];
        param -= lr * wd * param;
        float mm = beta1 * m[i] + (1.0f - beta1) * grad;
        float vv = beta2 * v[i] + (1.0f - beta2) * grad * grad;
        m[i] = mm;
        v[i] = vv;
        float m_hat = mm / bc1;
        float v_hat = vv / bc2;
        param -= lr * (m_hat / (sqrtf(v_hat) + eps));
        p[i] = param;
    }
}

float orc_clip_grad_norm(float* const* grads, const int64_t* sizes, int64_t count, float max_norm) {
    double tot = 0.0;
    for (int64_t t = 0; t < count; ++t) {
        double s = 0.0;
        for (int64_t i = 0; i < sizes[t]; ++i) s += (double)grads[t][i] * (double)grads[t][i];
        tot += s;
    }
    float norm = (float)sqrt(tot);
    float coef = max_norm / (norm + 1e-6f);
    if (coef < 1.0f)
        for (int64_t t = 0; t < count; ++t)
            for (int64_t i = 0; i < sizes[t]; ++i) grads[t][i] *= coef;
    return norm;
}

void orc_scaler_init(orc_scaler* s, float initial_scale, float growth_factor, float backoff_factor,
                     int growth_interval, float min_scale, float max_scale) {
    s->initial_scale = initial_scale;
    s->growth_factor = growth_factor;
    s->backoff_factor = backoff_factor;
    s->growth_interval = growth_interval;
    s->min_scale = min_scale;
    s->max_scale = max_scale;
    s->scale = initial_scale;
    s->good_steps = 0;
    s->skipped_steps = 0;
}

int orc_scaler_unscale_and_update(orc_scaler* s, float* const* grads, const int64_t* sizes, int64_t count) {
    for (int64_t t = 0; t < count; ++t)
        for (int64_t i = 0; i < sizes[t]; ++i)
            if (isnan(grads[t][i]) || isinf(grads[t][i])) {
                float ns = s->scale * s->backoff_factor;
                s->scale = ns > s->min_scale ? ns : s->min_scale;
                s->good_steps = 0;
                s->skipped_steps++;
                return 0;
            }
    float inv = 1.0f / s->scale;
    for (int64_t t = 0; t < count; ++t)
        for (int64_t i = 0; i < sizes[t]; ++i) grads[t][i] *= inv;
    s->good_steps++;
    if (s->good_steps >= s->growth_interval) {
        float ns = s->scale * s->growth_factor;
        s->scale = ns < s->max_scale ? ns : s->max_scale;
        s->good_steps = 0;
    }
    return 1;
}

/* ======================================================================================
 * TransformerLM step (src/models/transformer_lm.cpp:50-62, include/nn/transformer_block.hpp:26-36,
 * src/train/trainer.cpp:37-118 without the scheduler: lr is fixed)
 * ====================================================================================== */
typedef struct {
    float *wq, *wk, *wv, *wo, *wg, *wu, *wd, *n1, *n2;
    float *wr, *wex; /* MoE: router [E,d]; experts, each gate [f,d], up [f,d], down [d,f] */
} layer_ptrs;

typedef struct {
    float* emb;
    layer_ptrs* layers;
    float* normf;
    float* head;
} lm_ptrs;

/* QLoRA adapters of one layer (LoRALinear lora_A [r,in], lora_B [out,r]; src/nn/lora.cpp:31-43)
 * in the packed order of the trainable arena: A of q, k, v; B of q, k, v; A, B of out_proj; A of
 * gate, up; B of gate, up; A, B of down_proj. */
typedef struct {
    float *aq, *ak, *av, *bq, *bk, *bv, *ao, *bo, *ag, *au, *bg, *bu, *ad, *bd;
} lora_layer;

typedef struct {
    int64_t r;
    float s;        /* scaling alpha / r */
    lora_layer* P;  /* adapters */
    lora_layer* G;  /* their gradients */
} lora_ctx;

int64_t orc_qlora_num_params(const orc_lm_config* c, int64_t r) {
    int64_t d = c->d_model, f = c->d_ffn;
    return c->n_layers * (8 * r * d + 2 * (r * d + f * r) + r * f + d * r);
}

static lora_layer* map_lora(const orc_lm_config* c, int64_t r, float* base) {
    int64_t d = c->d_model, f = c->d_ffn;
    lora_layer* out = (lora_layer*)xcalloc((size_t)c->n_layers, sizeof(lora_layer));
    float* cur = base;
    for (int64_t l = 0; l < c->n_layers; ++l) {
        lora_layer* a = &out[l];
        a->aq = cur; cur += r * d;
        a->ak = cur; cur += r * d;
        a->av = cur; cur += r * d;
        a->bq = cur; cur += d * r;
        a->bk = cur; cur += d * r;
        a->bv = cur; cur += d * r;
        a->ao = cur; cur += r * d;
        a->bo = cur; cur += d * r;
        a->ag = cur; cur += r * d;
        a->au = cur; cur += r * d;
        a->bg = cur; cur += f * r;
        a->bu = cur; cur += f * r;
        a->ad = cur; cur += r * f;
        a->bd = cur; cur += d * r;
    }
    return out;
}

/* One projection y = x W^T, with LoRA when lc != NULL (LoRALinear::forward, lora.cpp:75-93). */
static void proj_fwd(const lora_ctx* lc, const float* x, const float* W, const float* A, const float* Bm, float* y,
                     int64_t B, int64_t S, int64_t in, int64_t out) {
    if (lc) orc_lora_fwd(x, W, A, Bm, lc->s, B, S, in, out, lc->r, y, NULL);
    else orc_linear_fwd(x, W, y, B, S, in, out);
}

/* Its backward: dW of a trainable base weight, or with LoRA dA/dB of the adapters and no base
 * gradient (the base is frozen). */
static void proj_bwd(const lora_ctx* lc, const float* x, const float* W, const float* A, const float* Bm,
                     const float* dy, float* dx, float* dW, float* dA, float* dB, int64_t B, int64_t S, int64_t in,
                     int64_t out) {
    if (lc) orc_lora_bwd(x, W, A, Bm, lc->s, dy, B, S, in, out, lc->r, dx, dA, dB);
    else orc_linear_bwd(x, W, dy, dx, dW, B, S, in, out);
}

int64_t orc_lm_num_params(const orc_lm_config* c) {
    int64_t d = c->d_model, f = c->d_ffn, V = c->vocab, E = c->n_experts;
    int64_t per_layer = 4 * d * d + (E > 0 ? E * d + E * 3 * d * f : 3 * d * f) + 2 * d;
    return V * d + c->n_layers * per_layer + d + (c->tied ? 0 : V * d);
}

static lm_ptrs map_params(const orc_lm_config* c, float* base) {
    lm_ptrs p;
    int64_t d = c->d_model, f = c->d_ffn, V = c->vocab;
    float* cur = base;
    p.emb = cur; cur += V * d;
    p.layers = (layer_ptrs*)xcalloc((size_t)c->n_layers, sizeof(layer_ptrs));
    for (int64_t l = 0; l < c->n_layers; ++l) {
        layer_ptrs* L = &p.layers[l];
        L->wq = cur; cur += d * d;
        L->wk = cur; cur += d * d;
        L->wv = cur; cur += d * d;
        L->wo = cur; cur += d * d;
        if (c->n_experts > 0) {
            L->wr = cur; cur += c->n_experts * d;
            L->wex = cur; cur += c->n_experts * 3 * f * d;
        } else {
            L->wg = cur; cur += f * d;
            L->wu = cur; cur += f * d;
            L->wd = cur; cur += d * f;
        }
        L->n1 = cur; cur += d;
        L->n2 = cur; cur += d;
    }
    p.normf = cur; cur += d;
    p.head = c->tied ? p.emb : cur;
    return p;
}

typedef struct {
    float *x, *h1, *r1, *q, *k, *v, *E, *rs, *ctx, *x1, *h2, *r2, *g, *u, *hm;
} layer_acts;

static void add_into(float* dst, const float* a, const float* b, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = a[i] + b[i];
}

/* Experts stored back to back (gate, up, down per expert) <-> the [E,f,d] / [E,d,f] stacks
 * the MoE restatement takes. */
static void experts_split(const float* wex, int64_t E, int64_t d, int64_t f, float* wg, float* wu, float* wd) {
    const int64_t fd = f * d;
    for (int64_t e = 0; e < E; ++e) {
        memcpy(wg + e * fd, wex + e * 3 * fd, sizeof(float) * (size_t)fd);
        memcpy(wu + e * fd, wex + e * 3 * fd + fd, sizeof(float) * (size_t)fd);
        memcpy(wd + e * fd, wex + e * 3 * fd + 2 * fd, sizeof(float) * (size_t)fd);
    }
}
static void experts_merge_add(float* wex, int64_t E, int64_t d, int64_t f, const float* wg, const float* wu,
                              const float* wd) {
    const int64_t fd = f * d;
    for (int64_t e = 0; e < E; ++e)
        for (int64_t i = 0; i < fd; ++i) {
            wex[e * 3 * fd + i] += wg[e * fd + i];
            wex[e * 3 * fd + fd + i] += wu[e * fd + i];
            wex[e * 3 * fd + 2 * fd + i] += wd[e * fd + i];
        }
}

static void moe_ffn_fwd_r(const float* h, const float* wr, const float* wg, const float* wu, const float* wd,
                          int64_t T, int64_t d, int64_t f, int64_t E, int64_t k, float aux_coef, const int64_t* forced,
                          float* y, float* aux, int64_t* idx_out, float* gates_out);
static void moe_ffn_bwd_r(const float* h, const float* wr, const float* wg, const float* wu, const float* wd,
                          int64_t T, int64_t d, int64_t f, int64_t E, int64_t k, float aux_coef, const int64_t* forced,
                          const float* dy, float daux, float* dh, float* dwr, float* dwg, float* dwu, float* dwd);

/* MoE routing of the LM step's layers (test control, orc_moe_set_routing): forced [L][T][k] top-k
 * selections used instead of each router's own (NULL: the routers decide), and out [L][T][k]
 * receiving the selections the forward used (NULL: not recorded). */
static const int64_t* g_moe_forced = NULL;
static int64_t* g_moe_out = NULL;
void orc_moe_set_routing(const int64_t* forced, int64_t* out) {
    g_moe_forced = forced;
    g_moe_out = out;
}

/* Forward; returns logits [T, V] (caller frees) and fills acts when non-NULL. */
static float* lm_forward(const orc_lm_config* c, const lm_ptrs* P, const int64_t* ids, int64_t B, int64_t S,
                         layer_acts* acts, float** hf_out, float** rf_out, float** xf_out,
                         const float* cos_t, const float* sin_t, orc_step_result* res, float* aux_total,
                         const lora_ctx* lc) {
    float aux_sum = 0.0f;
    int have_aux = 0;
    int64_t d = c->d_model, f = c->d_ffn, V = c->vocab, H = c->n_heads, hd = d / H, T = B * S;
    size_t Td = (size_t)(T * d), Tf = (size_t)(T * f);
    double t0 = now_s();
    float* x = (float*)xcalloc(Td, sizeof(float));
    orc_embedding_fwd(ids, P->emb, x, T, d, V);
    double t1 = now_s();
    for (int64_t l = 0; l < c->n_layers; ++l) {
        layer_ptrs* L = &P->layers[l];
        float* h1 = (float*)xcalloc(Td, sizeof(float));
        float* r1 = (float*)xcalloc((size_t)T, sizeof(float));
        float* q = (float*)xcalloc(Td, sizeof(float));
        float* k = (float*)xcalloc(Td, sizeof(float));
        float* v = (float*)xcalloc(Td, sizeof(float));
        float* ctx = (float*)xcalloc(Td, sizeof(float));
        float* att = (float*)xcalloc(Td, sizeof(float));
        float* x1 = (float*)xcalloc(Td, sizeof(float));
        float* h2 = (float*)xcalloc(Td, sizeof(float));
        float* r2 = (float*)xcalloc((size_t)T, sizeof(float));
        float* g = (float*)xcalloc(Tf, sizeof(float));
        float* u = (float*)xcalloc(Tf, sizeof(float));
        float* hm = (float*)xcalloc(Tf, sizeof(float));
        float* ffo = (float*)xcalloc(Td, sizeof(float));
        float* E = acts ? (float*)xcalloc((size_t)(B * H * S * S), sizeof(float)) : NULL;
        float* rs = acts ? (float*)xcalloc((size_t)(B * H * S), sizeof(float)) : NULL;

        const lora_layer* LA = lc ? &lc->P[l] : NULL;
        orc_rmsnorm_fwd(x, L->n1, h1, r1, T, d, c->norm_eps);
        proj_fwd(lc, h1, L->wq, LA ? LA->aq : NULL, LA ? LA->bq : NULL, q, B, S, d, d);
        proj_fwd(lc, h1, L->wk, LA ? LA->ak : NULL, LA ? LA->bk : NULL, k, B, S, d, d);
        proj_fwd(lc, h1, L->wv, LA ? LA->av : NULL, LA ? LA->bv : NULL, v, B, S, d, d);
        orc_rope_fwd(q, cos_t, sin_t, B, S, H, hd, 0);
        orc_rope_fwd(k, cos_t, sin_t, B, S, H, hd, 0);
        orc_attention_fwd(q, k, v, ctx, E, rs, B, S, H, hd, 1);
        proj_fwd(lc, ctx, L->wo, LA ? LA->ao : NULL, LA ? LA->bo : NULL, att, B, S, d, d);
        add_into(x1, x, att, (int64_t)Td);
        orc_rmsnorm_fwd(x1, L->n2, h2, r2, T, d, c->norm_eps);
        if (c->n_experts > 0) {
            /* MoETransformerBlock: x2 = x1 + MoELayer(norm2(x1)) (src/nn/moe.cpp:155-253, 283-300) */
            const int64_t E = c->n_experts;
            float* wg = (float*)xcalloc((size_t)(E * f * d), sizeof(float));
            float* wu = (float*)xcalloc((size_t)(E * f * d), sizeof(float));
            float* wd = (float*)xcalloc((size_t)(E * f * d), sizeof(float));
            experts_split(L->wex, E, d, f, wg, wu, wd);
            float aux = 0.0f;
            const int64_t lk = l * T * c->top_k;
            moe_ffn_fwd_r(h2, L->wr, wg, wu, wd, T, d, f, E, c->top_k, c->aux_coef,
                          g_moe_forced ? g_moe_forced + lk : NULL, ffo, &aux, g_moe_out ? g_moe_out + lk : NULL, NULL);
            aux_sum = have_aux ? aux_sum + aux : aux; /* total_aux_loss: add in layer order */
            have_aux = 1;
            free(wg); free(wu); free(wd);
        } else {
            proj_fwd(lc, h2, L->wg, LA ? LA->ag : NULL, LA ? LA->bg : NULL, g, B, S, d, f);
            proj_fwd(lc, h2, L->wu, LA ? LA->au : NULL, LA ? LA->bu : NULL, u, B, S, d, f);
            orc_swiglu_fwd(g, u, hm, (int64_t)Tf);
            proj_fwd(lc, hm, L->wd, LA ? LA->ad : NULL, LA ? LA->bd : NULL, ffo, B, S, f, d);
        }
        float* x2 = (float*)xcalloc(Td, sizeof(float));
        add_into(x2, x1, ffo, (int64_t)Td);
        free(att);
        free(ffo);
        if (acts) {
            layer_acts* A = &acts[l];
            A->x = x; A->h1 = h1; A->r1 = r1; A->q = q; A->k = k; A->v = v; A->E = E; A->rs = rs;
            A->ctx = ctx; A->x1 = x1; A->h2 = h2; A->r2 = r2; A->g = g; A->u = u; A->hm = hm;
        } else {
            free(x); free(h1); free(r1); free(q); free(k); free(v); free(ctx); free(x1); free(h2);
            free(r2); free(g); free(u); free(hm);
        }
        x = x2;
    }
    double t2 = now_s();
    float* hf = (float*)xcalloc(Td, sizeof(float));
    float* rf = (float*)xcalloc((size_t)T, sizeof(float));
    orc_rmsnorm_fwd(x, P->normf, hf, rf, T, d, c->norm_eps);
    float* logits = (float*)xcalloc((size_t)(T * V), sizeof(float));
    orc_linear_fwd(hf, P->head, logits, B, S, d, V);
    double t3 = now_s();
    if (res) {
        res->t_embed = t1 - t0;
        res->t_blocks_fwd = t2 - t1;
        res->t_head_fwd = t3 - t2;
    }
    if (hf_out) *hf_out = hf; else free(hf);
    if (rf_out) *rf_out = rf; else free(rf);
    if (xf_out) *xf_out = x; else free(x);
    if (aux_total) *aux_total = aux_sum;
    return logits;
}

float orc_lm_loss(const orc_lm_config* c, const float* params, const int64_t* ids, const int64_t* targets,
                  int64_t B, int64_t S) {
    lm_ptrs P = map_params(c, (float*)params);
    int64_t hd = c->d_model / c->n_heads;
    float* cos_t = (float*)xcalloc((size_t)(S * hd / 2), sizeof(float));
    float* sin_t = (float*)xcalloc((size_t)(S * hd / 2), sizeof(float));
    orc_rope_tables(cos_t, sin_t, S, hd, c->rope_base);
    float aux = 0.0f;
    float* logits = lm_forward(c, &P, ids, B, S, NULL, NULL, NULL, NULL, cos_t, sin_t, NULL, &aux, NULL);
    float loss = orc_ce_fwd(logits, targets, B * S, c->vocab, -100, NULL, NULL, NULL);
    if (c->n_experts > 0) loss = loss + aux;
    free(logits); free(cos_t); free(sin_t); free(P.layers);
    return loss;
}

/* The step on the dense parameters `params`; without LoRA (lc == NULL) the trainable tensors are
 * params themselves (gradients into grads), with LoRA they are the adapters of lc (trainable /
 * tgrads of nt elements) and params is the frozen base. */
static int lm_step_core(const orc_lm_config* c, float* params, float* grads, const lora_ctx* lc, float* trainable,
                        float* tgrads, int64_t nt, float* m, float* v, int64_t* step_count, const int64_t* ids,
                        const int64_t* targets, int64_t B, int64_t S, const orc_train_opts* o, orc_scaler* scaler,
                        orc_step_result* res) {
    orc_step_result local;
    if (!res) res = &local;
    memset(res, 0, sizeof(*res));
    if (S > c->max_seq_len) return -1;
    int64_t d = c->d_model, f = c->d_ffn, V = c->vocab, H = c->n_heads, hd = d / H, T = B * S;
    size_t Td = (size_t)(T * d), Tf = (size_t)(T * f);
    const int64_t np = nt;
    lm_ptrs P = map_params(c, params);
    memset(tgrads, 0, sizeof(float) * (size_t)nt);
    lm_ptrs G;
    if (grads) {
        G = map_params(c, grads);
    } else { /* frozen base: no gradient buffers */
        memset(&G, 0, sizeof(G));
        G.layers = (layer_ptrs*)xcalloc((size_t)c->n_layers, sizeof(layer_ptrs));
    }

    float* cos_t = (float*)xcalloc((size_t)(S * hd / 2), sizeof(float));
    float* sin_t = (float*)xcalloc((size_t)(S * hd / 2), sizeof(float));
    orc_rope_tables(cos_t, sin_t, S, hd, c->rope_base);

    layer_acts* acts = (layer_acts*)xcalloc((size_t)c->n_layers, sizeof(layer_acts));
    float *hf, *rf, *xf;
    float aux = 0.0f;
    float* logits = lm_forward(c, &P, ids, B, S, acts, &hf, &rf, &xf, cos_t, sin_t, res, &aux, lc);

    /* loss (+ total_aux_loss for MoE, tests/unit/test_moe.cpp:224-228) */
    double tl0 = now_s();
    float* lse = (float*)xcalloc((size_t)T, sizeof(float));
    int64_t valid = 0;
    float loss = orc_ce_fwd(logits, targets, T, V, -100, NULL, lse, &valid);
    if (c->n_experts > 0) loss = loss + aux;
    res->loss = loss;
    res->aux_loss = c->n_experts > 0 ? aux : 0.0f;
    float gscale = 1.0f;
    if (o->use_scaler && scaler) gscale = scaler->scale; /* scaler.scale(loss) = mul(loss, scale) */
    res->loss_scale_used = gscale;
    float* dlogits = (float*)xcalloc((size_t)(T * V), sizeof(float));
    orc_ce_bwd(logits, targets, lse, T, V, -100, valid, gscale, dlogits);
    free(logits);
    double tl1 = now_s();
    res->t_loss = tl1 - tl0;

    /* head + final norm backward */
    float* dh = (float*)xcalloc(Td, sizeof(float));
    orc_linear_bwd(hf, P.head, dlogits, dh, G.head, B, S, d, V);
    free(dlogits);
    float* dx = (float*)xcalloc(Td, sizeof(float));
    orc_rmsnorm_bwd(dh, xf, P.normf, rf, dx, G.normf, T, d);
    double tl2 = now_s();
    res->t_head_bwd = tl2 - tl1;

    /* blocks backward */
    float* tmp = (float*)xcalloc(Td, sizeof(float));
    float* tmp2 = (float*)xcalloc(Td, sizeof(float));
    float* dhm = (float*)xcalloc(Tf, sizeof(float));
    float* dg = (float*)xcalloc(Tf, sizeof(float));
    float* du = (float*)xcalloc(Tf, sizeof(float));
    float* dq = (float*)xcalloc(Td, sizeof(float));
    float* dk = (float*)xcalloc(Td, sizeof(float));
    float* dv = (float*)xcalloc(Td, sizeof(float));
    for (int64_t l = c->n_layers - 1; l >= 0; --l) {
        layer_ptrs* L = &P.layers[l];
        layer_ptrs* GL = &G.layers[l];
        layer_acts* A = &acts[l];
        const lora_layer* LA = lc ? &lc->P[l] : NULL;
        const lora_layer* LG = lc ? &lc->G[l] : NULL;
        if (c->n_experts > 0) {
            /* x2 = x1 + moe(h2); d loss / d aux_l = 1 (scaled with the loss) */
            const int64_t E = c->n_experts, efd = E * f * d;
            float* wg = (float*)xcalloc((size_t)efd, sizeof(float));
            float* wu = (float*)xcalloc((size_t)efd, sizeof(float));
            float* wd = (float*)xcalloc((size_t)efd, sizeof(float));
            float* dwg = (float*)xcalloc((size_t)efd, sizeof(float));
            float* dwu = (float*)xcalloc((size_t)efd, sizeof(float));
            float* dwd = (float*)xcalloc((size_t)efd, sizeof(float));
            experts_split(L->wex, E, d, f, wg, wu, wd);
            memset(tmp, 0, sizeof(float) * Td);
            moe_ffn_bwd_r(A->h2, L->wr, wg, wu, wd, T, d, f, E, c->top_k, c->aux_coef,
                          g_moe_forced ? g_moe_forced + l * T * c->top_k : NULL, dx, gscale, tmp, GL->wr, dwg, dwu,
                          dwd);
            experts_merge_add(GL->wex, E, d, f, dwg, dwu, dwd);
            free(wg); free(wu); free(wd); free(dwg); free(dwu); free(dwd);
        } else {
            /* x2 = x1 + down(hm): dx is grad of x2 */
            proj_bwd(lc, A->hm, L->wd, LA ? LA->ad : NULL, LA ? LA->bd : NULL, dx, dhm, GL->wd, LG ? LG->ad : NULL,
                     LG ? LG->bd : NULL, B, S, f, d);
            orc_swiglu_bwd(A->g, A->u, dhm, dg, du, (int64_t)Tf);
            proj_bwd(lc, A->h2, L->wg, LA ? LA->ag : NULL, LA ? LA->bg : NULL, dg, tmp, GL->wg, LG ? LG->ag : NULL,
                     LG ? LG->bg : NULL, B, S, d, f);
            proj_bwd(lc, A->h2, L->wu, LA ? LA->au : NULL, LA ? LA->bu : NULL, du, tmp2, GL->wu, LG ? LG->au : NULL,
                     LG ? LG->bu : NULL, B, S, d, f);
            add_into(tmp, tmp, tmp2, (int64_t)Td); /* grad of h2 (engine accumulation) */
        }
        orc_rmsnorm_bwd(tmp, A->x1, L->n2, A->r2, tmp2, GL->n2, T, d);
        add_into(dx, dx, tmp2, (int64_t)Td); /* grad of x1 = residual + norm path */
        /* x1 = x + out_proj(ctx) */
        proj_bwd(lc, A->ctx, L->wo, LA ? LA->ao : NULL, LA ? LA->bo : NULL, dx, tmp, GL->wo, LG ? LG->ao : NULL,
                 LG ? LG->bo : NULL, B, S, d, d);
        orc_attention_bwd(A->q, A->k, A->v, A->E, A->rs, tmp, dq, dk, dv, B, S, H, hd);
        orc_rope_bwd(dq, cos_t, sin_t, B, S, H, hd, 0);
        orc_rope_bwd(dk, cos_t, sin_t, B, S, H, hd, 0);
        proj_bwd(lc, A->h1, L->wq, LA ? LA->aq : NULL, LA ? LA->bq : NULL, dq, tmp, GL->wq, LG ? LG->aq : NULL,
                 LG ? LG->bq : NULL, B, S, d, d);
        proj_bwd(lc, A->h1, L->wk, LA ? LA->ak : NULL, LA ? LA->bk : NULL, dk, tmp2, GL->wk, LG ? LG->ak : NULL,
                 LG ? LG->bk : NULL, B, S, d, d);
        add_into(tmp, tmp, tmp2, (int64_t)Td);
        proj_bwd(lc, A->h1, L->wv, LA ? LA->av : NULL, LA ? LA->bv : NULL, dv, tmp2, GL->wv, LG ? LG->av : NULL,
                 LG ? LG->bv : NULL, B, S, d, d);
        add_into(tmp, tmp, tmp2, (int64_t)Td);
        orc_rmsnorm_bwd(tmp, A->x, L->n1, A->r1, tmp2, GL->n1, T, d);
        add_into(dx, dx, tmp2, (int64_t)Td);
        free(A->x); free(A->h1); free(A->r1); free(A->q); free(A->k); free(A->v); free(A->E); free(A->rs);
        free(A->ctx); free(A->x1); free(A->h2); free(A->r2); free(A->g); free(A->u); free(A->hm);
    }
    double tl3 = now_s();
    res->t_blocks_bwd = tl3 - tl2;
    if (G.emb) orc_embedding_bwd(ids, dx, G.emb, T, d, V);
    double tl4 = now_s();
    res->t_embed_bwd = tl4 - tl3;
    free(tmp); free(tmp2); free(dhm); free(dg); free(du); free(dq); free(dk); free(dv); free(dx); free(dh);
    free(hf); free(rf); free(xf); free(lse); free(acts); free(cos_t); free(sin_t);

    /* optimizer tail: [scaler] -> clip -> AdamW (src/train/trainer.cpp:70-95) */
    double to0 = now_s();
    float* gp[1] = {tgrads};
    int64_t gs[1] = {np};
    int ok = 1;
    if (o->use_scaler && scaler) ok = orc_scaler_unscale_and_update(scaler, gp, gs, 1);
    res->found_inf = !ok;
    if (ok) {
        if (o->max_grad_norm > 0.0f) {
            res->grad_norm = orc_clip_grad_norm(gp, gs, 1, o->max_grad_norm);
        } else {
            double s = 0.0;
            for (int64_t i = 0; i < np; ++i) s += (double)tgrads[i] * (double)tgrads[i];
            res->grad_norm = (float)sqrt(s);
        }
        if (o->do_update) {
            *step_count += 1;
            orc_adamw(trainable, tgrads, m, v, np, o->lr, o->beta1, o->beta2, o->eps, o->weight_decay, *step_count);
        }
    }
    res->t_optim = now_s() - to0;
    free(P.layers);
    free(G.layers);
    return 0;
}

/* TransformerLM::forward (src/models/transformer_lm.cpp:50-62): logits [B*S, V]. */
int orc_lm_logits(const orc_lm_config* c, const float* params, const int64_t* ids, int64_t B, int64_t S,
                  float* logits) {
    if (S > c->max_seq_len) return -1;
    lm_ptrs P = map_params(c, (float*)params);
    int64_t hd = c->d_model / c->n_heads;
    float* cos_t = (float*)xcalloc((size_t)(S * hd / 2), sizeof(float));
    float* sin_t = (float*)xcalloc((size_t)(S * hd / 2), sizeof(float));
    orc_rope_tables(cos_t, sin_t, S, hd, c->rope_base);
    float aux = 0.0f;
    float* l = lm_forward(c, &P, ids, B, S, NULL, NULL, NULL, NULL, cos_t, sin_t, NULL, &aux, NULL);
    memcpy(logits, l, sizeof(float) * (size_t)(B * S * c->vocab));
    free(l); free(cos_t); free(sin_t); free(P.layers);
    return 0;
}

int orc_lm_step(const orc_lm_config* c, float* params, float* grads, float* m, float* v, int64_t* step_count,
                const int64_t* ids, const int64_t* targets, int64_t B, int64_t S, const orc_train_opts* o,
                orc_scaler* scaler, orc_step_result* res) {
    return lm_step_core(c, params, grads, NULL, params, grads, orc_lm_num_params(c), m, v, step_count, ids, targets,
                        B, S, o, scaler, res);
}

/* QuantizedLinear::from_linear then forward's dequantization (src/nn/quantization.cpp:602-615,
 * 669-679) of the seven projections of every layer of the dense parameters, in place: INT4
 * symmetric groups of G with fp16 scales. */
int orc_qlora_dequantize_base(const orc_lm_config* c, int64_t G, float* params) {
    if (c->n_experts > 0) return -1;
    lm_ptrs P = map_params(c, params);
    const int64_t d = c->d_model, f = c->d_ffn;
    uint8_t* pk = (uint8_t*)xcalloc((size_t)(f * d / 2 + d * d / 2 + 1), 1);
    uint16_t* sc = (uint16_t*)xcalloc((size_t)((f * d + d * d) / G + 1), sizeof(uint16_t));
    int rc = 0;
    for (int64_t l = 0; l < c->n_layers && rc == 0; ++l) {
        layer_ptrs* L = &P.layers[l];
        float* w[7] = {L->wq, L->wk, L->wv, L->wo, L->wg, L->wu, L->wd};
        const int64_t n[7] = {d * d, d * d, d * d, d * d, f * d, f * d, d * f};
        for (int j = 0; j < 7 && rc == 0; ++j) {
            rc = orc_int4_quantize(w[j], n[j], G, 1, pk, sc);
            if (rc == 0) rc = orc_int4_dequantize(pk, sc, 1, n[j], G, w[j]);
        }
    }
    free(pk);
    free(sc);
    free(P.layers);
    return rc;
}

/* The QLoRA step: base (dense layout) is frozen; its projections are the INT4 round trip of
 * orc_qlora_dequantize_base, done here on a copy; only the adapters `lora` are trained. */
int orc_qlora_step(const orc_lm_config* c, int64_t r, float alpha, int64_t G, const float* base, float* lora,
                   float* grads, float* m, float* v, int64_t* step_count, const int64_t* ids, const int64_t* targets,
                   int64_t B, int64_t S, const orc_train_opts* o, orc_scaler* scaler, orc_step_result* res) {
    if (c->n_experts > 0 || r <= 0) return -1;
    const int64_t np = orc_lm_num_params(c), nl = orc_qlora_num_params(c, r);
    float* w = (float*)xcalloc((size_t)np, sizeof(float));
    memcpy(w, base, sizeof(float) * (size_t)np);
    int rc = orc_qlora_dequantize_base(c, G, w);
    if (rc == 0) {
        lora_ctx lc;
        lc.r = r;
        lc.s = alpha / (float)r;
        lc.P = map_lora(c, r, lora);
        memset(grads, 0, sizeof(float) * (size_t)nl);
        lc.G = map_lora(c, r, grads);
        rc = lm_step_core(c, w, NULL, &lc, lora, grads, nl, m, v, step_count, ids, targets, B, S, o, scaler, res);
        free(lc.P);
        free(lc.G);
    }
    free(w);
    return rc;
}

/* ======================================================================================
 * Mixture of experts (src/nn/moe.cpp)
 * ====================================================================================== */

/* Row softmax as the reference composes it (src/ops/ops.cpp:460-471): m = max (no gradient),
 * ex = exp(x - m), s = sum(ex) accumulated in double, p = ex / s. */
static void softmax_row(const float* x, float* p, int64_t n) {
    float m = x[0];
    for (int64_t i = 1; i < n; ++i) m = x[i] > m ? x[i] : m;
    double s = 0.0;
    for (int64_t i = 0; i < n; ++i) {
        p[i] = expf(x[i] - m);
        s += (double)p[i];
    }
    const float sf = (float)s;
    for (int64_t i = 0; i < n; ++i) p[i] = p[i] / sf;
}

/* Backward of softmax_row through its div / sum / exp ops (src/autograd/functions.cpp):
 * dx = p * (dp - sum(dp * p)), the reduction in double.  Adds into dx. */
static void softmax_row_bwd(const float* p, const float* dp, float* dx, int64_t n) {
    double s = 0.0;
    for (int64_t i = 0; i < n; ++i) s += (double)dp[i] * (double)p[i];
    const float sf = (float)s;
    for (int64_t i = 0; i < n; ++i) dx[i] += p[i] * (dp[i] - sf);
}

/* MoERouter::route (moe.cpp:33-129) and the gate normalisation of MoELayer::forward
 * (moe.cpp:170-204) on precomputed gate logits [T,E]:
 *   probs = softmax(logits); idx[t, 0..k) = the k largest logits, descending, ties broken by the
 *   lower expert index (the reference's std::partial_sort leaves tie order unspecified; this
 *   explicit rule is the one the kernel implements); rweights = softmax over the selected logits
 *   with the 1e-9 of moe.cpp:74; counts[e] = tokens routed to e; mean_probs = mean_t probs (double
 *   sum); aux = sum_e mean_probs[e] * counts[e] * E * coef / (T * k) when coef > 0 and E > 1,
 *   else 0; gates = probs * mask / (sum(probs * mask) + 1e-9).  Any output may be NULL. */
static void moe_route_r(const float* logits, int64_t T, int64_t E, int64_t k, float aux_coef, const int64_t* forced,
                        int64_t* idx, float* rweights, float* gates, float* probs, int64_t* counts, float* mean_probs,
                        float* aux);
void orc_moe_route(const float* logits, int64_t T, int64_t E, int64_t k, float aux_coef, int64_t* idx,
                   float* rweights, float* gates, float* probs, int64_t* counts, float* mean_probs, float* aux) {
    moe_route_r(logits, T, E, k, aux_coef, NULL, idx, rweights, gates, probs, counts, mean_probs, aux);
}

/* The same with the selection given: forced [T,k] (k distinct experts per token, in order) when
 * not NULL -- test control, so that a step can be compared on another implementation's routing;
 * every other quantity (probabilities, gates, counts, aux) follows from it as above. */
static void moe_route_r(const float* logits, int64_t T, int64_t E, int64_t k, float aux_coef, const int64_t* forced,
                        int64_t* idx, float* rweights, float* gates, float* probs, int64_t* counts, float* mean_probs,
                        float* aux) {
    float* p = (float*)xcalloc((size_t)(T * E), sizeof(float));
    int64_t* cnt = (int64_t*)xcalloc((size_t)E, sizeof(int64_t));
    int64_t* sel = (int64_t*)xcalloc((size_t)k, sizeof(int64_t));
    char* used = (char*)xcalloc((size_t)E, 1);
    for (int64_t t = 0; t < T; ++t) {
        const float* row = logits + t * E;
        softmax_row(row, p + t * E, E);
        memset(used, 0, (size_t)E);
        for (int64_t j = 0; j < k; ++j) { /* selection: largest remaining logit, lowest index on ties */
            int64_t best = -1;
            if (forced) {
                best = forced[t * k + j];
            } else {
                for (int64_t e = 0; e < E; ++e)
                    if (!used[e] && (best < 0 || row[e] > row[best])) best = e;
            }
            used[best] = 1;
            sel[j] = best;
            cnt[best]++;
            if (idx) idx[t * k + j] = best;
        }
        if (rweights) {
            const float mx = row[sel[0]];
            float se = 0.0f;
            for (int64_t j = 0; j < k; ++j) se += expf(row[sel[j]] - mx);
            for (int64_t j = 0; j < k; ++j) rweights[t * k + j] = expf(row[sel[j]] - mx) / (se + 1e-9f);
        }
        if (gates) {
            /* masked = probs * mask; denom = sum(masked, -1) + 1e-9 (sum in double) */
            double s = 0.0;
            for (int64_t e = 0; e < E; ++e) s += used[e] ? (double)p[t * E + e] : 0.0;
            const float den = (float)s + 1e-9f;
            for (int64_t e = 0; e < E; ++e) gates[t * E + e] = (used[e] ? p[t * E + e] : 0.0f) / den;
        }
    }
    double auxd = 0.0;
    const float scale = ((float)E * aux_coef) / ((float)T * (float)k);
    for (int64_t e = 0; e < E; ++e) {
        double s = 0.0;
        for (int64_t t = 0; t < T; ++t) s += (double)p[t * E + e];
        const float mp = (float)(s / (double)T);
        if (mean_probs) mean_probs[e] = mp;
        if (counts) counts[e] = cnt[e];
        auxd += (double)(mp * ((float)cnt[e] * scale));
    }
    if (aux) *aux = (aux_coef > 0.0f && E > 1) ? (float)auxd : 0.0f;
    if (probs) memcpy(probs, p, sizeof(float) * (size_t)(T * E));
    free(used);
    free(sel);
    free(cnt);
    free(p);
}

/* Tokens routed to expert e, in token order. */
static int64_t moe_rows(const int64_t* idx, int64_t T, int64_t k, int64_t e, int64_t* rows) {
    int64_t n = 0;
    for (int64_t t = 0; t < T; ++t)
        for (int64_t j = 0; j < k; ++j)
            if (idx[t * k + j] == e) rows[n++] = t;
    return n;
}

/* MoELayer::forward (moe.cpp:155-253) on the normalised input h [T,d]: router weights wr [E,d],
 * experts e: gate wg[e] [f,d], up wu[e] [f,d], down wd[e] [d,f] (SwiGLU, include/nn/swiglu.hpp).
 * y[t] = sum over the selected experts in increasing e of gates[t,e] * SwiGLU_e(h[t]); the
 * reference evaluates every active expert on all tokens and multiplies by a zero gate for the
 * unrouted ones, which adds exact zeros, so the sparse sum is the same.  Outputs idx [T,k],
 * gates [T,E] and aux may be NULL. */
static void moe_ffn_fwd_r(const float* h, const float* wr, const float* wg, const float* wu, const float* wd,
                          int64_t T, int64_t d, int64_t f, int64_t E, int64_t k, float aux_coef, const int64_t* forced,
                          float* y, float* aux, int64_t* idx_out, float* gates_out);
void orc_moe_ffn_fwd(const float* h, const float* wr, const float* wg, const float* wu, const float* wd, int64_t T,
                     int64_t d, int64_t f, int64_t E, int64_t k, float aux_coef, float* y, float* aux, int64_t* idx_out,
                     float* gates_out) {
    moe_ffn_fwd_r(h, wr, wg, wu, wd, T, d, f, E, k, aux_coef, NULL, y, aux, idx_out, gates_out);
}
/* forced: the top-k selection to use (moe_route_r), NULL for the router's own. */
static void moe_ffn_fwd_r(const float* h, const float* wr, const float* wg, const float* wu, const float* wd,
                          int64_t T, int64_t d, int64_t f, int64_t E, int64_t k, float aux_coef, const int64_t* forced,
                          float* y, float* aux, int64_t* idx_out, float* gates_out) {
    float* logits = (float*)xcalloc((size_t)(T * E), sizeof(float));
    orc_linear_fwd(h, wr, logits, 1, T, d, E);
    int64_t* idx = (int64_t*)xcalloc((size_t)(T * k), sizeof(int64_t));
    float* gates = (float*)xcalloc((size_t)(T * E), sizeof(float));
    moe_route_r(logits, T, E, k, aux_coef, forced, idx, NULL, gates, NULL, NULL, NULL, aux);
    memset(y, 0, sizeof(float) * (size_t)(T * d));
    int64_t* rows = (int64_t*)xcalloc((size_t)T, sizeof(int64_t));
    float* xe = (float*)xcalloc((size_t)(T * d), sizeof(float));
    float* g = (float*)xcalloc((size_t)(T * f), sizeof(float));
    float* u = (float*)xcalloc((size_t)(T * f), sizeof(float));
    float* a = (float*)xcalloc((size_t)(T * f), sizeof(float));
    float* ye = (float*)xcalloc((size_t)(T * d), sizeof(float));
    for (int64_t e = 0; e < E; ++e) {
        const int64_t n = moe_rows(idx, T, k, e, rows);
        if (n == 0) continue;
        for (int64_t r = 0; r < n; ++r) memcpy(xe + r * d, h + rows[r] * d, sizeof(float) * (size_t)d);
        orc_linear_fwd(xe, wg + e * f * d, g, 1, n, d, f);
        orc_linear_fwd(xe, wu + e * f * d, u, 1, n, d, f);
        orc_swiglu_fwd(g, u, a, n * f);
        orc_linear_fwd(a, wd + e * d * f, ye, 1, n, f, d);
        for (int64_t r = 0; r < n; ++r) {
            const float gt = gates[rows[r] * E + e];
            for (int64_t c = 0; c < d; ++c) y[rows[r] * d + c] += ye[r * d + c] * gt;
        }
    }
    if (idx_out) memcpy(idx_out, idx, sizeof(int64_t) * (size_t)(T * k));
    if (gates_out) memcpy(gates_out, gates, sizeof(float) * (size_t)(T * E));
    free(ye); free(a); free(u); free(g); free(xe); free(rows); free(gates); free(idx); free(logits);
}

/* Backward of orc_moe_ffn_fwd for dL/dy = dy and dL/daux = daux, through the reference's graph:
 * mul (expert output x gate column, the broadcast reduction in double), the expert SwiGLUs, the
 * gate normalisation (div / sum / add 1e-9), the mask, both router softmaxes (the one of route()
 * feeding mean_probs and the aux loss, the one of forward() feeding the gates) and both gate
 * Linear applications.  Gradients are added into dh [T,d], dwr [E,d], dwg/dwu [E,f,d], dwd [E,d,f]. */
static void moe_ffn_bwd_r(const float* h, const float* wr, const float* wg, const float* wu, const float* wd,
                          int64_t T, int64_t d, int64_t f, int64_t E, int64_t k, float aux_coef, const int64_t* forced,
                          const float* dy, float daux, float* dh, float* dwr, float* dwg, float* dwu, float* dwd);
void orc_moe_ffn_bwd(const float* h, const float* wr, const float* wg, const float* wu, const float* wd, int64_t T,
                     int64_t d, int64_t f, int64_t E, int64_t k, float aux_coef, const float* dy, float daux, float* dh,
                     float* dwr, float* dwg, float* dwu, float* dwd) {
    moe_ffn_bwd_r(h, wr, wg, wu, wd, T, d, f, E, k, aux_coef, NULL, dy, daux, dh, dwr, dwg, dwu, dwd);
}
static void moe_ffn_bwd_r(const float* h, const float* wr, const float* wg, const float* wu, const float* wd,
                          int64_t T, int64_t d, int64_t f, int64_t E, int64_t k, float aux_coef, const int64_t* forced,
                          const float* dy, float daux, float* dh, float* dwr, float* dwg, float* dwu, float* dwd) {
    float* logits = (float*)xcalloc((size_t)(T * E), sizeof(float));
    orc_linear_fwd(h, wr, logits, 1, T, d, E);
    int64_t* idx = (int64_t*)xcalloc((size_t)(T * k), sizeof(int64_t));
    float* gates = (float*)xcalloc((size_t)(T * E), sizeof(float));
    float* probs = (float*)xcalloc((size_t)(T * E), sizeof(float));
    int64_t* counts = (int64_t*)xcalloc((size_t)E, sizeof(int64_t));
    moe_route_r(logits, T, E, k, aux_coef, forced, idx, NULL, gates, probs, counts, NULL, NULL);
    float* dgates = (float*)xcalloc((size_t)(T * E), sizeof(float));
    int64_t* rows = (int64_t*)xcalloc((size_t)T, sizeof(int64_t));
    float* xe = (float*)xcalloc((size_t)(T * d), sizeof(float));
    float* g = (float*)xcalloc((size_t)(T * f), sizeof(float));
    float* u = (float*)xcalloc((size_t)(T * f), sizeof(float));
    float* a = (float*)xcalloc((size_t)(T * f), sizeof(float));
    float* ye = (float*)xcalloc((size_t)(T * d), sizeof(float));
    float* dye = (float*)xcalloc((size_t)(T * d), sizeof(float));
    float* da = (float*)xcalloc((size_t)(T * f), sizeof(float));
    float* dg = (float*)xcalloc((size_t)(T * f), sizeof(float));
    float* du = (float*)xcalloc((size_t)(T * f), sizeof(float));
    float* dxe = (float*)xcalloc((size_t)(T * d), sizeof(float));
    float* dxe2 = (float*)xcalloc((size_t)(T * d), sizeof(float));
    for (int64_t e = 0; e < E; ++e) {
        const int64_t n = moe_rows(idx, T, k, e, rows);
        if (n == 0) continue; /* inactive experts are skipped: no gradient at all */
        for (int64_t r = 0; r < n; ++r) memcpy(xe + r * d, h + rows[r] * d, sizeof(float) * (size_t)d);
        orc_linear_fwd(xe, wg + e * f * d, g, 1, n, d, f);
        orc_linear_fwd(xe, wu + e * f * d, u, 1, n, d, f);
        orc_swiglu_fwd(g, u, a, n * f);
        orc_linear_fwd(a, wd + e * d * f, ye, 1, n, f, d);
        for (int64_t r = 0; r < n; ++r) {
            const int64_t t = rows[r];
            const float gt = gates[t * E + e];
            double s = 0.0;
            for (int64_t c = 0; c < d; ++c) {
                dye[r * d + c] = dy[t * d + c] * gt;
                s += (double)(dy[t * d + c] * ye[r * d + c]);
            }
            dgates[t * E + e] = (float)s;
        }
        orc_linear_bwd(a, wd + e * d * f, dye, da, dwd + e * d * f, 1, n, f, d);
        orc_swiglu_bwd(g, u, da, dg, du, n * f);
        orc_linear_bwd(xe, wg + e * f * d, dg, dxe, dwg + e * f * d, 1, n, d, f);
        orc_linear_bwd(xe, wu + e * f * d, du, dxe2, dwu + e * f * d, 1, n, d, f);
        for (int64_t r = 0; r < n; ++r)
            for (int64_t c = 0; c < d; ++c) dh[rows[r] * d + c] += dxe[r * d + c] + dxe2[r * d + c];
    }
    /* router: gates = masked / (sum(masked) + 1e-9), masked = probs * mask */
    float* dlogits = (float*)xcalloc((size_t)(T * E), sizeof(float));
    float* dp = (float*)xcalloc((size_t)E, sizeof(float));
    const float fscale = ((float)E * aux_coef) / ((float)T * (float)k);
    const int aux_on = aux_coef > 0.0f && E > 1;
    for (int64_t t = 0; t < T; ++t) {
        double den_d = 0.0;
        char used[256] = {0};
        for (int64_t j = 0; j < k; ++j) used[idx[t * k + j]] = 1;
        for (int64_t e = 0; e < E; ++e) den_d += used[e] ? (double)probs[t * E + e] : 0.0;
        const float den = (float)den_d + 1e-9f;
        double sb = 0.0; /* grad of the denominator: sum_e -dg * masked / den^2 */
        for (int64_t e = 0; e < E; ++e) {
            const float masked = used[e] ? probs[t * E + e] : 0.0f;
            sb += (double)(-dgates[t * E + e] * masked / (den * den));
        }
        for (int64_t e = 0; e < E; ++e) dp[e] = used[e] ? (dgates[t * E + e] / den + (float)sb) : 0.0f;
        softmax_row_bwd(probs + t * E, dp, dlogits + t * E, E);
        if (aux_on) { /* route()'s softmax: d mean_probs[e] = daux * f_e, mean over T */
            for (int64_t e = 0; e < E; ++e) dp[e] = (daux * ((float)counts[e] * fscale)) / (float)T;
            softmax_row_bwd(probs + t * E, dp, dlogits + t * E, E);
        }
    }
    float* dhr = (float*)xcalloc((size_t)(T * d), sizeof(float));
    orc_linear_bwd(h, wr, dlogits, dhr, dwr, 1, T, d, E);
    for (int64_t i = 0; i < T * d; ++i) dh[i] += dhr[i];
    free(dhr); free(dp); free(dlogits);
    free(dxe2); free(dxe); free(du); free(dg); free(da); free(dye); free(ye); free(a); free(u); free(g); free(xe);
    free(rows); free(dgates); free(counts); free(probs); free(gates); free(idx); free(logits);
}

/* ======================================================================================
 * INT4 symmetric quantization (src/nn/quantization.cpp:197-295 quantize, :359-474 dequantize,
 * include/nn/quantization.hpp:41-56 nibble packing)
 * ====================================================================================== */

/* IEEE binary32 -> binary16, round to nearest even, subnormals kept (the fp16 scale storage
 * of the QLoRA configuration; the reference stores fp32 scales). */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, sizeof x);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to infinity */
    const int e = (int)(ax >> 23) - 127;
    if (e >= -14) {
        const uint32_t m = ax & 0x7fffffu, rem = m & 0x1fffu;
        uint32_t h = ((uint32_t)(e + 15) << 10) | (m >> 13);
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u; /* a carry bumps the exponent */
        return (uint16_t)(sign | h);
    }
    if (e < -25) return (uint16_t)sign;
    const uint32_t m = (ax & 0x7fffffu) | 0x800000u; /* |f| = m * 2^(e-23); unit 2^-24 */
    const int sh = -(e + 1);                         /* 14..24 */
    const uint32_t rem = m & ((1u << sh) - 1u), halfw = 1u << (sh - 1);
    uint32_t h = m >> sh;
    if (rem > halfw || (rem == halfw && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

float orc_f16_to_f32(uint16_t h) {
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    float v;
    if (e == 0) v = ldexpf((float)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexpf((float)(m | 0x400u), (int)e - 25);
    return (h & 0x8000u) ? -v : v;
}

static float int4_scale(const void* scales, int scale_f16, int64_t g) {
    return scale_f16 ? orc_f16_to_f32(((const uint16_t*)scales)[g]) : ((const float*)scales)[g];
}

int orc_int4_quantize(const float* x, int64_t n, int64_t G, int scale_f16, uint8_t* packed, void* scales) {
    if (n < 0) return 1;
    if (n == 0) return 0;
    if (G <= 0 || G > n) G = n; /* group_size <= 0: one group over the tensor (quantization.cpp:202-205) */
    const int64_t ng = (n + G - 1) / G;
    if (ng > 1 && (G & 1)) return 2; /* odd groups would share a byte between two groups */
    memset(packed, 0, (size_t)((n + 1) / 2));
    for (int64_t g = 0; g < ng; ++g) {
        const int64_t start = g * G, end = start + G < n ? start + G : n;
        float amax = fabsf(x[start]);
        for (int64_t i = start + 1; i < end; ++i) {
            const float av = fabsf(x[i]);
            if (av > amax) amax = av;
        }
        float s = amax / 7.0f;
        if (s < 1e-8f) s = 1e-8f;
        if (scale_f16) ((uint16_t*)scales)[g] = orc_f32_to_f16(s);
        else ((float*)scales)[g] = s;
        for (int64_t i = start; i < end; i += 2) {
            float q0 = roundf(x[i] / s); /* std::round: halves away from zero */
            q0 = q0 < -7.0f ? -7.0f : (q0 > 7.0f ? 7.0f : q0);
            int q1i = 0;
            if (i + 1 < end) {
                float q1 = roundf(x[i + 1] / s);
                q1 = q1 < -7.0f ? -7.0f : (q1 > 7.0f ? 7.0f : q1);
                q1i = (int)q1;
            }
            packed[i / 2] = (uint8_t)(((unsigned)(q1i & 0x0f) << 4) | ((unsigned)((int)q0) & 0x0fu));
        }
    }
    return 0;
}

int orc_int4_dequantize(const uint8_t* packed, const void* scales, int scale_f16, int64_t n, int64_t G, float* out) {
    if (n < 0) return 1;
    if (n == 0) return 0;
    if (G <= 0 || G > n) G = n;
    if ((n + G - 1) / G > 1 && (G & 1)) return 2;
    for (int64_t i = 0; i < n; ++i) {
        const unsigned b = packed[i / 2], u = (i & 1) ? (b >> 4) : (b & 0x0fu);
        const int q = u >= 8 ? (int)u - 16 : (int)u;
        out[i] = (float)q * int4_scale(scales, scale_f16, i / G);
    }
    return 0;
}

/* The CUDA launcher's general INT4 dequantization (src/cuda/cuda_quantize.cu:54-94, 141-159): per
 * element i, the nibble u (low nibble of byte i/2 for even i, high for odd), val = u - 16 when
 * is_signed and u >= 8, else u; g = i / G (G <= 0: group 0); out = (val - zp[g]) * s[g] in fp32,
 * zp = 0 without zero points.  Any G, odd ones included (each element finds its own group). */
int orc_int4_dequantize_zp(const uint8_t* packed, const float* scales, const float* zp, int is_signed, int64_t n,
                           int64_t G, float* out) {
    if (n < 0) return 1;
    for (int64_t i = 0; i < n; ++i) {
        const unsigned b = packed[i / 2], u = (i & 1) ? ((b >> 4) & 0x0fu) : (b & 0x0fu);
        const float val = (is_signed && u >= 8) ? (float)((int)u - 16) : (float)u;
        const int64_t g = G > 0 ? i / G : 0;
        const float z = zp ? zp[g] : 0.0f;
        out[i] = (val - z) * scales[g];
    }
    return 0;
}

/* ======================================================================================
 * LoRA (src/nn/lora.cpp:31-108)
 * ====================================================================================== */

void orc_lora_fwd(const float* x, const float* W, const float* A, const float* Bm, float scaling, int64_t Bt,
                  int64_t S, int64_t in, int64_t out, int64_t r, float* y, float* xa_out) {
    const int64_t T = Bt * S;
    float* xa = (float*)xcalloc((size_t)(T * r), sizeof(float));
    float* lo = (float*)xcalloc((size_t)(T * out), sizeof(float));
    orc_linear_fwd(x, W, y, Bt, S, in, out);
    orc_linear_fwd(x, A, xa, Bt, S, in, r);
    orc_linear_fwd(xa, Bm, lo, Bt, S, r, out);
    for (int64_t i = 0; i < T * out; ++i) y[i] = y[i] + lo[i] * scaling;
    if (xa_out) memcpy(xa_out, xa, sizeof(float) * (size_t)(T * r));
    free(lo);
    free(xa);
}

void orc_lora_bwd(const float* x, const float* W, const float* A, const float* Bm, float scaling, const float* dy,
                  int64_t Bt, int64_t S, int64_t in, int64_t out, int64_t r, float* dx, float* dA, float* dB) {
    const int64_t T = Bt * S;
    float* xa = (float*)xcalloc((size_t)(T * r), sizeof(float));
    float* dl = (float*)xcalloc((size_t)(T * out), sizeof(float));
    float* dxa = (float*)xcalloc((size_t)(T * r), sizeof(float));
    float* dxl = (float*)xcalloc((size_t)(T * in), sizeof(float));
    orc_linear_fwd(x, A, xa, Bt, S, in, r);
    for (int64_t i = 0; i < T * out; ++i) dl[i] = dy[i] * scaling; /* MulBackward of lora_out * scaling */
    orc_linear_bwd(xa, Bm, dl, dxa, dB, Bt, S, r, out);
    orc_linear_bwd(x, A, dxa, dx ? dxl : NULL, dA, Bt, S, in, r);
    if (dx) {
        orc_linear_bwd(x, W, dy, dx, NULL, Bt, S, in, out); /* frozen base: no dW */
        for (int64_t i = 0; i < T * in; ++i) dx[i] = dx[i] + dxl[i];
    }
    free(dxl);
    free(dxa);
    free(dl);
    free(xa);
}

void orc_lora_merge(float* W, const float* A, const float* Bm, float scaling, int64_t in, int64_t out, int64_t r,
                    int sign) {
    float* dw = (float*)xcalloc((size_t)(out * in), sizeof(float));
    orc_gemm(Bm, A, dw, out, in, r);
    for (int64_t i = 0; i < out * in; ++i) {
        const float d = dw[i] * scaling;
        W[i] = sign >= 0 ? W[i] + d : W[i] - d;
    }
    free(dw);
}

/* ======================================================================================
 * Tensor primitives (src/ops/cpu_ops.cpp, src/tensor/tensor.cpp, src/core/shape.cpp,
 * src/ops/ops.cpp cat, src/autograd/functions.cpp reduce_gradient_for_broadcast)
 * ====================================================================================== */

/* Shape::broadcast (src/core/shape.cpp:138-166); returns the output rank or -1. */
int orc_broadcast_shape(const int64_t* a, int ra, const int64_t* b, int rb, int64_t* out) {
    const int r = ra > rb ? ra : rb;
    for (int i = 0; i < r; ++i) {
        const int64_t da = i < ra ? a[ra - 1 - i] : 1, db = i < rb ? b[rb - 1 - i] : 1;
        if (da != db && da != 1 && db != 1) return -1;
        out[r - 1 - i] = da > db ? da : db;
    }
    return r;
}

/* Shape::broadcast_strides (src/core/shape.cpp:168-195); returns 0 or -1. */
static int bcast_strides(const int64_t* shape, const int64_t* strides, int r, const int64_t* target, int tr,
                         int64_t* out) {
    if (r > tr) return -1;
    for (int i = 0; i < tr; ++i) {
        const int oi = r - 1 - i, ti = tr - 1 - i;
        if (oi >= 0) {
            if (shape[oi] == target[ti]) out[ti] = strides[oi];
            else if (shape[oi] == 1) out[ti] = 0;
            else return -1;
        } else {
            out[ti] = 0;
        }
    }
    return 0;
}

/* Tensor::clone of a strided view (src/tensor/tensor.cpp:255-297): row-major multi-index walk. */
void orc_strided_copy(const void* src, int64_t offset, int ndim, const int64_t* shape, const int64_t* strides,
                      int64_t elem_size, void* dst) {
    int64_t total = 1, coords[16] = {0};
    for (int i = 0; i < ndim; ++i) total *= shape[i];
    const char* s = (const char*)src;
    char* d = (char*)dst;
    for (int64_t lin = 0; lin < total; ++lin) {
        int64_t off = offset;
        for (int i = 0; i < ndim; ++i) off += coords[i] * strides[i];
        memcpy(d + lin * elem_size, s + off * elem_size, (size_t)elem_size);
        for (int i = ndim - 1; i >= 0; --i) {
            if (++coords[i] < shape[i]) break;
            coords[i] = 0;
        }
    }
}

/* float_to_half / half_to_float / float_to_bf16 (include/core/dtype.hpp:65-133), restated. */
static uint16_t ref_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t mant = x & 0x007FFFFFu;
    const int32_t exp = (int32_t)((x >> 23) & 0xFFu);
    if (exp == 0xFF) return (uint16_t)(sign | 0x7C00u | (mant ? (0x200u | (mant >> 13)) : 0u));
    const int32_t e = exp - 127 + 15;
    if (e >= 0x1F) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        mant |= 0x00800000u;
        const uint32_t shift = (uint32_t)(14 - e);
        uint32_t hm = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u), halfway = 1u << (shift - 1u);
        if (rem > halfway || (rem == halfway && (hm & 1u))) ++hm;
        return (uint16_t)(sign | hm);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)h;
}

static uint16_t ref_f32_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7F800000u) == 0x7F800000u && (x & 0x007FFFFFu) != 0) return (uint16_t)(((x >> 16) & 0x8000u) | 0x7FC0u);
    return (uint16_t)((x + 0x7FFFu + ((x >> 16) & 1u)) >> 16);
}

static float ref_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16, exp = (h >> 10) & 0x1Fu;
    uint32_t mant = h & 0x3FFu, bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            int e = -1;
            do {
                ++e;
                mant <<= 1;
            } while ((mant & 0x400u) == 0);
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((mant & 0x3FFu) << 13);
        }
    } else if (exp == 0x1F) {
        bits = sign | 0x7F800000u | (mant << 13);  /* NaN payloads are kept as they are */
    } else {
        bits = sign | ((exp + 112u) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static float ref_bf16_to_f32(uint16_t b) {
    const uint32_t x = (uint32_t)b << 16;
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* Tensor::to(DType) cast table (src/tensor/tensor.cpp:359-410).  dtype codes as aic::DType:
 * 0 f32, 1 f16, 2 bf16, 3 i32, 4 i64.  Returns 0, or 1 for a pair the reference rejects. */
int orc_cast(const void* src, int from, void* dst, int to, int64_t n) {
    if (from == to) {
        const int64_t es = (from == 4) ? 8 : ((from == 0 || from == 3) ? 4 : 2);
        memcpy(dst, src, (size_t)(n * es));
        return 0;
    }
    for (int64_t i = 0; i < n; ++i) {
        if (from == 0 && to == 1) ((uint16_t*)dst)[i] = ref_f32_to_f16(((const float*)src)[i]);
        else if (from == 0 && to == 2) ((uint16_t*)dst)[i] = ref_f32_to_bf16(((const float*)src)[i]);
        else if (from == 1 && to == 0) ((float*)dst)[i] = ref_f16_to_f32(((const uint16_t*)src)[i]);
        else if (from == 2 && to == 0) ((float*)dst)[i] = ref_bf16_to_f32(((const uint16_t*)src)[i]);
        else if (from == 0 && to == 4) ((int64_t*)dst)[i] = (int64_t)((const float*)src)[i];
        else if (from == 4 && to == 0) ((float*)dst)[i] = (float)((const int64_t*)src)[i];
        else if (from == 0 && to == 3) ((int32_t*)dst)[i] = (int32_t)((const float*)src)[i];
        else if (from == 3 && to == 0) ((float*)dst)[i] = (float)((const int32_t*)src)[i];
        else if (from == 4 && to == 3) ((int32_t*)dst)[i] = (int32_t)((const int64_t*)src)[i];
        else if (from == 3 && to == 4) ((int64_t*)dst)[i] = (int64_t)((const int32_t*)src)[i];
        else return 1;
    }
    return 0;
}

/* binary_broadcast_cpu (src/ops/cpu_ops.cpp:14-60); op 0 add, 1 sub, 2 mul, 3 div.  Views are
 * (offset, shape, strides) in elements; out is contiguous of the broadcast shape.  Returns 0 or -1. */
int orc_binary(int op, const float* a, int64_t a_off, const int64_t* a_shape, const int64_t* a_strides, int ra,
               const float* b, int64_t b_off, const int64_t* b_shape, const int64_t* b_strides, int rb, float* out) {
    int64_t oshape[16], sa[16], sb[16], coords[16] = {0};
    const int r = orc_broadcast_shape(a_shape, ra, b_shape, rb, oshape);
    if (r < 0 || bcast_strides(a_shape, a_strides, ra, oshape, r, sa) || bcast_strides(b_shape, b_strides, rb, oshape, r, sb))
        return -1;
    int64_t total = 1;
    for (int i = 0; i < r; ++i) total *= oshape[i];
    for (int64_t lin = 0; lin < total; ++lin) {
        int64_t oa = a_off, ob = b_off;
        for (int k = 0; k < r; ++k) {
            oa += coords[k] * sa[k];
            ob += coords[k] * sb[k];
        }
        const float x = a[oa], y = b[ob];
        out[lin] = op == 0 ? x + y : (op == 1 ? x - y : (op == 2 ? x * y : x / y));
        for (int k = r - 1; k >= 0; --k) {
            if (++coords[k] < oshape[k]) break;
            coords[k] = 0;
        }
    }
    return 0;
}

/* unary_cpu functions (src/ops/cpu_ops.cpp:105-146): 0 neg, 1 abs, 2 exp, 3 log, 4 sqrt, 5 tanh,
 * 6 sigmoid, 7 gelu (tanh form), 8 silu. */
void orc_unary(int op, const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        const float v = x[i];
        float r;
        switch (op) {
            case 0: r = -v; break;
            case 1: r = fabsf(v); break;
            case 2: r = expf(v); break;
            case 3: r = logf(v); break;
            case 4: r = sqrtf(v); break;
            case 5: r = tanhf(v); break;
            case 6: r = 1.0f / (1.0f + expf(-v)); break;
            case 7: {
                const float inner = 0.7978845608f * (v + 0.044715f * v * v * v);
                r = 0.5f * v * (1.0f + tanhf(inner));
                break;
            }
            default: r = v / (1.0f + expf(-v)); break;
        }
        y[i] = r;
    }
}

/* Full reductions (src/ops/cpu_ops.cpp:151-197): 0 sum (double), 1 mean (sum / (float)n),
 * 2 max, 3 min (NaN never replaces the running value). */
float orc_reduce_all(int op, const float* x, int64_t n) {
    if (op == 0 || op == 1) {
        double acc = 0.0;
        for (int64_t i = 0; i < n; ++i) acc += (double)x[i];
        float s = (float)acc;
        if (op == 1) s /= (float)n;
        return s;
    }
    float m = op == 2 ? -INFINITY : INFINITY;
    for (int64_t i = 0; i < n; ++i)
        if (op == 2 ? x[i] > m : x[i] < m) m = x[i];
    return m;
}

/* reduce_dim_cpu (src/ops/cpu_ops.cpp:203-271) on a contiguous x of `shape`: out has the shape
 * without `dim` (keepdim only changes the shape).  Mean is (float)(sum / size) in double. */
void orc_reduce_dim(int op, const float* x, int ndim, const int64_t* shape, int dim, float* out) {
    int64_t outer = 1, inner = 1;
    for (int i = 0; i < dim; ++i) outer *= shape[i];
    for (int i = dim + 1; i < ndim; ++i) inner *= shape[i];
    const int64_t rs = shape[dim];
    for (int64_t o = 0; o < outer; ++o)
        for (int64_t in = 0; in < inner; ++in) {
            const float* p = x + o * rs * inner + in;
            double acc = 0.0;
            float mx = -INFINITY, mn = INFINITY;
            for (int64_t k = 0; k < rs; ++k) {
                const float v = p[k * inner];
                if (op <= 1) acc += (double)v;
                else if (op == 2) { if (v > mx) mx = v; }
                else if (v < mn) mn = v;
            }
            out[o * inner + in] = op == 0 ? (float)acc : (op == 1 ? (float)(acc / (double)rs) : (op == 2 ? mx : mn));
        }
}

/* cat along `dim` of `count` contiguous inputs that agree outside dim (src/ops/ops.cpp:473-530):
 * out = [outer, sum(mid_i), inner]. */
void orc_cat(const void* const* srcs, const int64_t* mids, int count, int64_t outer, int64_t inner, int64_t elem_size,
             void* dst) {
    int64_t total_mid = 0;
    for (int i = 0; i < count; ++i) total_mid += mids[i];
    int64_t off = 0;
    for (int i = 0; i < count; ++i) {
        const int64_t row = mids[i] * inner * elem_size;
        for (int64_t o = 0; o < outer; ++o)
            memcpy((char*)dst + (o * total_mid + off) * inner * elem_size, (const char*)srcs[i] + o * row, (size_t)row);
        off += mids[i];
    }
}

/* reduce_gradient_for_broadcast (src/autograd/functions.cpp:10-41): sum over leading dims, then
 * over the dims where the target has size 1 (each a reduce_dim sum, rounded to float between
 * steps).  out has the target's element count.  Returns 0 or -1. */
int orc_sum_to_shape(const float* g, int ndim, const int64_t* shape, int tr, const int64_t* target, float* out) {
    int64_t cur[16], n = 1;
    int r = ndim;
    for (int i = 0; i < ndim; ++i) { cur[i] = shape[i]; n *= shape[i]; }
    float* buf = (float*)xcalloc((size_t)(n > 0 ? n : 1), sizeof(float));
    float* tmp = (float*)xcalloc((size_t)(n > 0 ? n : 1), sizeof(float));
    memcpy(buf, g, sizeof(float) * (size_t)n);
    if (tr == 0) {
        out[0] = orc_reduce_all(0, buf, n);
        free(tmp); free(buf);
        return 0;
    }
    while (r > tr) {
        orc_reduce_dim(0, buf, r, cur, 0, tmp);
        n /= cur[0];
        for (int i = 0; i + 1 < r; ++i) cur[i] = cur[i + 1];
        --r;
        float* t = buf; buf = tmp; tmp = t;
    }
    for (int i = 0; i < tr; ++i) {
        if (target[i] == 1 && cur[i] > 1) {
            orc_reduce_dim(0, buf, r, cur, i, tmp);
            n /= cur[i];
            cur[i] = 1;
            float* t = buf; buf = tmp; tmp = t;
        }
    }
    for (int i = 0; i < tr; ++i)
        if (cur[i] != target[i]) { free(tmp); free(buf); return -1; }
    memcpy(out, buf, sizeof(float) * (size_t)n);
    free(tmp);
    free(buf);
    return 0;
}
