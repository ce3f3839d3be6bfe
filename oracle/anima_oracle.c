/*
 * anima_oracle.c -- CPU oracle for the Anima DiT attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker: tests, the smoke
 * check and the benchmark's CPU-baseline leg call it to produce expected
 * values.  The product library (libanima_hip.so) never links, loads or calls
 * it, and no product code path falls back to it.
 *
 * Each function restates one function of the reference runtime (anima_rt) in
 * plain C, keeping the reference's arithmetic order exactly so that results
 * are bit-identical to the reference built with `g++ -O2` on x86-64 (no FMA
 * contraction: this file is compiled with -ffp-contract=off, and the
 * reference's baseline x86-64 build has no FMA instructions either).
 *
 * Pinning (what checks each function independently of this restatement):
 *   oracle_flash_attention  -- bit-identical to the reference build in
 *       oracle/_ref (anima_rt_run_sdpa_flash), fp64 brute-force SDPA,
 *       closed-form invariants (Sk=1 -> O=V, Q=0 -> mean(V), convexity).
 *   oracle_sdpa_math        -- bit-identical to oracle/_ref anima_rt_run_sdpa;
 *       fp64 SDPA evaluated at scale^2.
 *   oracle_rmsnorm          -- bit-identical to oracle/_ref anima_rt_run_rmsnorm;
 *       fp64 closed form.
 *   oracle_rope             -- bit-identical to oracle/_ref anima_rt_run_rope;
 *       the D=4 known-answer test of scripts/test_rope_debug.py:17-34;
 *       norm preservation per rotated pair.
 *   oracle_gemm_bf16        -- fp64 GEMM on the bf16-decoded weights.
 *   oracle_layernorm        -- bit-identical to oracle/_ref anima_rt_run_layernorm;
 *       fp64 two-pass mean/variance.
 *   oracle_silu             -- bit-identical to oracle/_ref anima_rt_run_silu;
 *       fp64 x / (1 + exp(-x)).
 *   oracle_softmax          -- bit-identical to oracle/_ref anima_rt_run_softmax;
 *       fp64 exp(x - max) / sum, rows summing to 1.
 *   oracle_gelu             -- bit-identical to oracle/_ref anima_rt_run_gelu;
 *       fp64 x * Phi(x) via math.erf; GELU(0) = 0, GELU(x) - GELU(-x) = x.
 *   oracle_modulate, oracle_gate_residual -- numpy float32 evaluation of the
 *       same expressions (each operation rounded to float32).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <pthread.h>

/* Query/key tile sizes of anima_rt's flash attention
 * (anima_rt/include/cpu/flash_attention.h:62-67). */
static int q_split_for(int S_q)
{
    int q = (S_q >= 768) ? 256 : (S_q >= 192) ? 64 : 32;
    return q > S_q ? S_q : q;
}

/* One (batch*head) slice of the flash attention.  Follows
 * anima_rt/include/cpu/flash_attention.h:84-202 for a single bh:
 * scores = (serial dot) * scale, -inf padding, causal mask, per-row online
 * max/sum update with the rescale applied only for kvStart > 0, P.V axpy that
 * skips exact zeros, final multiply by 1/sum. */
static void flash_one_head(const float *Qh, const float *Kh, const float *Vh,
                           float *Oh, int S_q, int S_kv, int D, float scale,
                           int is_causal, float *scores, float *mx, float *sm)
{
    const int qs = q_split_for(S_q);
    const int kvs = S_kv < 512 ? S_kv : 512;
    for (int q0 = 0; q0 < S_q; q0 += qs) {
        const int nq = (q0 + qs <= S_q) ? qs : (S_q - q0);
        for (int r = 0; r < nq; r++) {
            mx[r] = -INFINITY;
            sm[r] = 0.0f;
            memset(Oh + (int64_t)(q0 + r) * D, 0, sizeof(float) * (size_t)D);
        }
        const int nkeys = is_causal ? ((q0 + nq < S_kv) ? q0 + nq : S_kv) : S_kv;
        for (int k0 = 0; k0 < S_kv; k0 += kvs) {
            const int nk = (k0 + kvs <= S_kv) ? kvs : (S_kv - k0);
            if (k0 >= nkeys)
                break;
            int live = nk;
            if (is_causal) {
                if (nkeys - k0 < nk)
                    live = nkeys - k0;
                if (live <= 0)
                    break;
            }
            for (int i = 0; i < nq; i++) {
                const float *qrow = Qh + (int64_t)(q0 + i) * D;
                float *srow = scores + (int64_t)i * nk;
                for (int j = 0; j < live; j++) {
                    const float *krow = Kh + (int64_t)(k0 + j) * D;
                    float acc = 0.0f;
                    for (int d = 0; d < D; d++)
                        acc += qrow[d] * krow[d];
                    srow[j] = acc * scale;
                }
                for (int j = live; j < nk; j++)
                    srow[j] = -INFINITY;
            }
            if (is_causal) {
                for (int i = 0; i < nq; i++)
                    for (int j = 0; j < nk; j++)
                        if (k0 + j > q0 + i)
                            scores[(int64_t)i * nk + j] = -INFINITY;
            }
            for (int i = 0; i < nq; i++) {
                float *srow = scores + (int64_t)i * nk;
                float *orow = Oh + (int64_t)(q0 + i) * D;
                float tmax = -INFINITY;
                for (int j = 0; j < nk; j++)
                    if (srow[j] > tmax)
                        tmax = srow[j];
                if (tmax == -INFINITY)
                    continue;
                const float m_new = (mx[i] > tmax) ? mx[i] : tmax;
                const float alpha = (mx[i] == -INFINITY) ? 0.0f : expf(mx[i] - m_new);
                if (k0 > 0)
                    for (int d = 0; d < D; d++)
                        orow[d] *= alpha;
                sm[i] = sm[i] * alpha;
                float tsum = 0.0f;
                for (int j = 0; j < nk; j++) {
                    const float e = expf(srow[j] - m_new);
                    srow[j] = e;
                    tsum += e;
                }
                sm[i] += tsum;
                for (int j = 0; j < nk; j++) {
                    const float p = srow[j];
                    if (p == 0.0f)
                        continue;
                    const float *vrow = Vh + (int64_t)(k0 + j) * D;
                    for (int d = 0; d < D; d++)
                        orow[d] += p * vrow[d];
                }
                mx[i] = m_new;
            }
        }
        for (int i = 0; i < nq; i++) {
            if (sm[i] > 0.0f) {
                const float inv = 1.0f / sm[i];
                float *orow = Oh + (int64_t)(q0 + i) * D;
                for (int d = 0; d < D; d++)
                    orow[d] *= inv;
            }
        }
    }
}

struct flash_job {
    const float *Q, *K, *V;
    float *O;
    int bh_begin, bh_end, S_q, S_kv, D, is_causal;
    float scale;
    int ok;
};

static void *flash_worker(void *arg)
{
    struct flash_job *j = (struct flash_job *)arg;
    const int qs = q_split_for(j->S_q);
    const int kvs = j->S_kv < 512 ? j->S_kv : 512;
    float *scores = (float *)malloc(sizeof(float) * (size_t)qs * (size_t)kvs + 16);
    float *mx = (float *)malloc(sizeof(float) * (size_t)qs + 16);
    float *sm = (float *)malloc(sizeof(float) * (size_t)qs + 16);
    j->ok = scores && mx && sm;
    if (j->ok) {
        for (int bh = j->bh_begin; bh < j->bh_end; bh++) {
            flash_one_head(j->Q + (int64_t)bh * j->S_q * j->D,
                           j->K + (int64_t)bh * j->S_kv * j->D,
                           j->V + (int64_t)bh * j->S_kv * j->D,
                           j->O + (int64_t)bh * j->S_q * j->D,
                           j->S_q, j->S_kv, j->D, j->scale, j->is_causal,
                           scores, mx, sm);
        }
    }
    free(scores);
    free(mx);
    free(sm);
    return NULL;
}

/* anima_rt_run_sdpa_flash (anima_rt/src/anima_rt.cpp:147-156) ->
 * anima::cpu::flash_attention (flash_attention.h:55-208).
 * Q,O: [BH,S_q,D]; K,V: [BH,S_kv,D]; contiguous fp32.  Single-threaded,
 * like the reference.  Returns 1 on success. */
int oracle_flash_attention(const float *Q, const float *K, const float *V,
                           float *O, int BH, int S_q, int S_kv, int D,
                           float scale, int is_causal)
{
    if (BH <= 0 || S_q <= 0 || S_kv <= 0 || D <= 0)
        return 1;
    struct flash_job j = {Q, K, V, O, 0, BH, S_q, S_kv, D, is_causal, scale, 0};
    flash_worker(&j);
    return j.ok;
}

/* The same computation with the independent (batch*head) slices spread over
 * `nthreads` POSIX threads.  Every slice runs the single-threaded code above,
 * so results are bit-identical to oracle_flash_attention. */
int oracle_flash_attention_mt(const float *Q, const float *K, const float *V,
                              float *O, int BH, int S_q, int S_kv, int D,
                              float scale, int is_causal, int nthreads)
{
    if (BH <= 0 || S_q <= 0 || S_kv <= 0 || D <= 0)
        return 1;
    if (nthreads > BH)
        nthreads = BH;
    if (nthreads <= 1)
        return oracle_flash_attention(Q, K, V, O, BH, S_q, S_kv, D, scale, is_causal);
    struct flash_job *jobs = (struct flash_job *)calloc((size_t)nthreads, sizeof(*jobs));
    pthread_t *tid = (pthread_t *)calloc((size_t)nthreads, sizeof(*tid));
    if (!jobs || !tid) {
        free(jobs);
        free(tid);
        return 0;
    }
    int ok = 1;
    for (int t = 0; t < nthreads; t++) {
        jobs[t] = (struct flash_job){Q, K, V, O, (int)((int64_t)BH * t / nthreads),
                                     (int)((int64_t)BH * (t + 1) / nthreads),
                                     S_q, S_kv, D, is_causal, scale, 0};
        if (pthread_create(&tid[t], NULL, flash_worker, &jobs[t]) != 0) {
            flash_worker(&jobs[t]);
            tid[t] = 0;
        }
    }
    for (int t = 0; t < nthreads; t++) {
        if (tid[t])
            pthread_join(tid[t], NULL);
        ok = ok && jobs[t].ok;
    }
    free(jobs);
    free(tid);
    return ok;
}

/* anima_rt "math" SDPA (anima_rt/src/anima_rt.cpp:78-141).  Both Q and K are
 * multiplied by `scale` (:95-98), so the result is softmax(scale^2 Q K^T) V.
 * GEMM = sgemm_fallback (anima_rt/src/gemm_backend.cpp:101-114), softmax =
 * softmax_kernel (anima_rt/include/cpu/softmax_kernel.h:14-41), A.V = the
 * manual loop at anima_rt.cpp:126-133.  Returns 0 on allocation failure. */
int oracle_sdpa_math(const float *Q, const float *K, const float *V, float *O,
                     int BH, int S_q, int S_kv, int D, float scale, int is_causal)
{
    const int64_t nq = (int64_t)BH * S_q * D, nk = (int64_t)BH * S_kv * D;
    float *qs = (float *)malloc(sizeof(float) * (size_t)(nq + 1));
    float *ks = (float *)malloc(sizeof(float) * (size_t)(nk + 1));
    float *att = (float *)malloc(sizeof(float) * ((size_t)S_q * (size_t)S_kv + 1));
    if (!qs || !ks || !att) {
        free(qs);
        free(ks);
        free(att);
        return 0;
    }
    for (int64_t i = 0; i < nq; i++)
        qs[i] = Q[i] * scale;
    for (int64_t i = 0; i < nk; i++)
        ks[i] = K[i] * scale;
    for (int h = 0; h < BH; h++) {
        const float *qh = qs + (int64_t)h * S_q * D;
        const float *kh = ks + (int64_t)h * S_kv * D;
        const float *vh = V + (int64_t)h * S_kv * D;
        float *oh = O + (int64_t)h * S_q * D;
        for (int i = 0; i < S_q; i++)
            for (int j = 0; j < S_kv; j++) {
                float acc = 0.0f;
                for (int d = 0; d < D; d++)
                    acc += qh[(int64_t)i * D + d] * kh[(int64_t)j * D + d];
                att[(int64_t)i * S_kv + j] = acc;
            }
        if (is_causal)
            for (int i = 0; i < S_q; i++)
                for (int j = 0; j < S_kv; j++)
                    att[(int64_t)i * S_kv + j] += (j > i) ? -INFINITY : 0.0f;
        for (int i = 0; i < S_q; i++) {
            float *row = att + (int64_t)i * S_kv;
            float m = row[0];
            for (int j = 1; j < S_kv; j++)
                if (row[j] > m)
                    m = row[j];
            float s = 0.0f;
            for (int j = 0; j < S_kv; j++) {
                const float e = expf(row[j] - m);
                row[j] = e;
                s += e;
            }
            const float inv = 1.0f / s;
            for (int j = 0; j < S_kv; j++)
                row[j] *= inv;
        }
        for (int i = 0; i < S_q; i++)
            for (int d = 0; d < D; d++) {
                float acc = 0.0f;
                for (int j = 0; j < S_kv; j++)
                    acc += att[(int64_t)i * S_kv + j] * vh[(int64_t)j * D + d];
                oh[(int64_t)i * D + d] = acc;
            }
    }
    free(qs);
    free(ks);
    free(att);
    return 1;
}

/* RMSNorm (anima_rt/include/cpu/rmsnorm_kernel.h:11-31): serial fp32 sum of
 * squares, 1/sqrt(sum/D + eps), times the optional weight. */
void oracle_rmsnorm(const float *X, const float *w, float *Y, int64_t M,
                    int64_t D, float eps)
{
    for (int64_t r = 0; r < M; r++) {
        const float *x = X + r * D;
        float *y = Y + r * D;
        float ss = 0.0f;
        for (int64_t j = 0; j < D; j++)
            ss += x[j] * x[j];
        const float inv = 1.0f / sqrtf(ss / (float)D + eps);
        for (int64_t j = 0; j < D; j++) {
            float v = x[j] * inv;
            if (w)
                v *= w[j];
            y[j] = v;
        }
    }
}

/* Rotate-half RoPE (anima_rt/include/cpu/rope_kernel.h:65-97): pairs (p, p+D/2)
 * with the 2x2 entry [c00,c01;c10,c11] of freqs[s][p], laid out [S][D/2][2][2].
 *   out[p]     = c00*x[p] + c01*x[p+D/2]
 *   out[p+D/2] = c10*x[p] + c11*x[p+D/2]
 * t,out: [N,S,D]. */
void oracle_rope(const float *t, const float *freqs, float *out, int N, int S, int D)
{
    const int half = D / 2;
    for (int n = 0; n < N; n++)
        for (int s = 0; s < S; s++) {
            const float *x = t + ((int64_t)n * S + s) * D;
            float *y = out + ((int64_t)n * S + s) * D;
            const float *f = freqs + (int64_t)s * D * 2;
            for (int p = 0; p < half; p++) {
                const float a = x[p], b = x[half + p];
                y[p] = f[4 * p + 0] * a + f[4 * p + 1] * b;
                y[half + p] = f[4 * p + 2] * a + f[4 * p + 3] * b;
            }
        }
}

/* fp32 -> bf16 round-to-nearest-even (anima_rt/src/gemm_backend.cpp:77-85). */
uint16_t oracle_f32_to_bf16(float f)
{
    uint32_t bits;
    memcpy(&bits, &f, sizeof(bits));
    bits += 0x7FFFu + ((bits >> 16) & 1u);
    return (uint16_t)(bits >> 16);
}

/* C[M,N] = A[M,K] . W[N,K]^T with W stored as bf16
 * (anima_rt/src/gemm_backend.cpp:117-131, sbgemm_fallback). */
void oracle_gemm_bf16(const float *A, const uint16_t *W, float *C, int M, int N, int K)
{
    for (int i = 0; i < M; i++)
        for (int j = 0; j < N; j++) {
            const float *a = A + (int64_t)i * K;
            const uint16_t *w = W + (int64_t)j * K;
            float acc = 0.0f;
            for (int k = 0; k < K; k++) {
                uint32_t bits = ((uint32_t)w[k]) << 16;
                float wf;
                memcpy(&wf, &bits, sizeof(wf));
                acc += a[k] * wf;
            }
            C[(int64_t)i * N + j] = acc;
        }
}

/* LayerNorm without affine parameters, as anima_rt_run_layernorm calls it
 * (anima_rt/src/anima_rt.cpp:36-43 -> layernorm_kernel,
 * anima_rt/include/cpu/layernorm_kernel.h:13-33): Welford moments
 * (anima_rt/include/cpu/welford.h:15-31, one correctly rounded divide per
 * step), population variance, rstd = 1/sqrt(var + eps), y = (x - mean)*rstd. */
void oracle_layernorm(const float *X, float *Y, int64_t M, int64_t D, float eps)
{
    for (int64_t r = 0; r < M; r++) {
        const float *x = X + r * D;
        float *y = Y + r * D;
        float mean = 0.0f, m2 = 0.0f;
        int64_t count = 0;
        for (int64_t i = 0; i < D; i++) {
            const float v = x[i];
            count++;
            const float delta = v - mean;
            mean += delta / (float)count;
            const float delta2 = v - mean;
            m2 += delta * delta2;
        }
        const float var = count > 0 ? m2 / (float)count : 0.0f;
        const float rstd = 1.0f / sqrtf(var + eps);
        for (int64_t j = 0; j < D; j++)
            y[j] = (x[j] - mean) * rstd;
    }
}

/* SiLU (anima_rt/include/cpu/silu_kernel.h:11-20): x / (1 + exp(-x)). */
void oracle_silu(const float *x, float *y, int64_t n)
{
    for (int64_t i = 0; i < n; i++)
        y[i] = x[i] / (1.0f + expf(-x[i]));
}

/* GELU, exact erf form (anima_rt/include/cpu/gelu_kernel.h:13-23):
 * x * 0.5 * (1 + erf(x * (float)M_SQRT1_2)), evaluated left to right. */
void oracle_gelu(const float *x, float *y, int64_t n)
{
    const float alpha = 0.70710678118654752440f;
    for (int64_t i = 0; i < n; i++) {
        const float h = x[i] * 0.5f;
        y[i] = h * (1.0f + erff(x[i] * alpha));
    }
}

/* Softmax over the last axis (anima_rt/include/cpu/softmax_kernel.h:16-40):
 * max by strict comparison from the first element, exp(x - max) stored and
 * summed in order, then multiplied by 1/sum. */
void oracle_softmax(const float *X, float *Y, int64_t outer, int64_t dim)
{
    for (int64_t i = 0; i < outer; i++) {
        const float *x = X + i * dim;
        float *y = Y + i * dim;
        float mx = x[0];
        for (int64_t j = 1; j < dim; j++)
            if (x[j] > mx)
                mx = x[j];
        float sum = 0.0f;
        for (int64_t j = 0; j < dim; j++) {
            const float v = expf(x[j] - mx);
            y[j] = v;
            sum += v;
        }
        const float inv = 1.0f / sum;
        for (int64_t j = 0; j < dim; j++)
            y[j] *= inv;
    }
}

/* AdaLN modulation of NumpyBlock.forward (anima_rt/scripts/numpy_dit.py:238,
 * 244, 250), x_m = x_n*(1.0 + scale) + shift in float32, with per-batch
 * vectors: x_n [B, S, D], scale/shift [B, D]. */
void oracle_modulate(const float *xn, const float *scale, const float *shift, float *y,
                     int B, int64_t S, int64_t D)
{
    for (int b = 0; b < B; b++)
        for (int64_t s = 0; s < S; s++)
            for (int64_t d = 0; d < D; d++) {
                const int64_t i = ((int64_t)b * S + s) * D + d;
                const float t = 1.0f + scale[(int64_t)b * D + d];
                const float m = xn[i] * t;
                y[i] = m + shift[(int64_t)b * D + d];
            }
}

/* Gated residual of NumpyBlock.forward (numpy_dit.py:240, 246, 252),
 * x = x + gate*out in float32, per-batch gate [B, D]; x updated in place. */
void oracle_gate_residual(float *x, const float *gate, const float *out, int B, int64_t S,
                          int64_t D)
{
    for (int b = 0; b < B; b++)
        for (int64_t s = 0; s < S; s++)
            for (int64_t d = 0; d < D; d++) {
                const int64_t i = ((int64_t)b * S + s) * D + d;
                const float g = gate[(int64_t)b * D + d] * out[i];
                x[i] = x[i] + g;
            }
}
