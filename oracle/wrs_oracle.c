/*
 * CPU oracle for the whisper.rs attention path -- TEST INFRASTRUCTURE ONLY.
 *
 * A C restatement of the reference's CPU algorithm. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load this library,
 * and only as the parity reference / timed baseline. The product library never links
 * or calls it.
 *
 * Reference files restated here (paths relative to the reference root):
 *   crates/tensor/src/ops/attention.rs   flash_attention_2, multi_head_attention,
 *                                        single_token_mha_d64 (AVX2 and scalar)
 *   crates/tensor/src/ops/softmax.rs     softmax_inplace
 *   crates/tensor/src/simd.rs:4-119      dot_f32 (AVX2+FMA and scalar)
 *   crates/whisper/src/decoder.rs:835-892 multi_head_attention_with_cache
 *   crates/whisper/src/decoder.rs:796-828 capture_cross_attention_heads
 *   crates/tensor/src/simd.rs:593-700    dot_f16_f32 (AVX2+F16C and scalar)
 *   crates/tensor/src/ops/quant.rs:343-473 f16_linear (LinearWeight::linear
 *                                        with f16 weights, weight.rs:116-137)
 *   crates/tensor/src/ops/norm.rs:1-143  layer_norm (AVX2 and scalar rows)
 *   crates/tensor/src/ops/gelu.rs:1-23   gelu_scalar, gelu_inplace
 *   crates/tensor/tests/test_flash_attention_tiled.rs:15-35 xorshift32 inputs
 *
 * What pins each function (checked in tests/test_oracle.py):
 *   softmax_inplace        closed forms (uniform row, one-hot limit, shift
 *                          invariance), sum-to-one, f64 brute force.
 *   dot_f32                f64 brute force (|err| bound), exact small-integer
 *                          inputs, AVX2 body == scalar body on exact inputs.
 *   flash_attention_2      every known-answer test of
 *                          crates/tensor/tests/test_flash_attention_tiled.rs and
 *                          crates/tensor/tests/test_flash_attention.rs against a
 *                          materialized f64 softmax (1e-5 / 1e-4), tile
 *                          boundaries, causal clamps, the stale-NaN sentinel,
 *                          K==0 -> mean of V rows, one dominant key -> its
 *                          value row, key-permutation invariance.
 *   single_token_mha_d64   same materialized reference (1e-5), AVX2 body vs
 *                          scalar body, softmax-weights of 1e-7 skip rule.
 *   mha_with_cache         materialized causal-with-offset reference; n=1
 *                          dispatch equals single_token_mha_d64 bitwise.
 *   capture_cross_heads    f64 softmax of the head's scores (1e-6) with the
 *                          [row][slot][n_audio] placement, the reference
 *                          test's row checks (test_dtw_alignment.rs:60-74),
 *                          K == 0 -> exactly fl(1/n_audio), dominant key,
 *                          and weights x V == multi_head_attention per head.
 * Bitwise equality with the Rust binary is NOT pinned for the tiled path: the
 * reference's two matrix products run in matrixmultiply 0.3.11 sgemm
 * (Cargo.lock:257-260), which is not vendored under the reference tree. Its
 * published micro-kernel accumulates each output with sequential FMAs over the
 * contraction index and then applies alpha/beta, which is what sgemm_tile()
 * below does; the reference's own tests only bound it to 1e-5.
 *
 * Build: oracle/Makefile (gcc, -ffp-contract=off so that no multiply-add is
 * fused unless the reference fuses it explicitly).
 */
#include "wrs_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#if defined(__x86_64__)
#include <immintrin.h>
#define WRS_HAVE_X86 1
#else
#define WRS_HAVE_X86 0
#endif

static int g_force_scalar = 0;

void wrs_oracle_force_scalar(int on) { g_force_scalar = on ? 1 : 0; }

int wrs_oracle_uses_avx2(void) {
#if WRS_HAVE_X86
    if (g_force_scalar) return 0;
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
#else
    return 0;
#endif
}

/* ------------------------------------------------------------------------ */
/* softmax.rs:1-23                                                           */
/* ------------------------------------------------------------------------ */
void wrs_oracle_softmax_inplace(float *x, size_t n) {
    if (n == 0) return;
    float max_val = -INFINITY;
    for (size_t i = 0; i < n; ++i)
        if (x[i] > max_val) max_val = x[i]; /* `if x > max_val` (:8) */
    float sum = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        x[i] = expf(x[i] - max_val);
        sum += x[i];
    }
    float inv_sum = 1.0f / sum; /* reciprocal multiply, :19-22 */
    for (size_t i = 0; i < n; ++i) x[i] *= inv_sum;
}

/* ------------------------------------------------------------------------ */
/* simd.rs dot_f32                                                           */
/* ------------------------------------------------------------------------ */
static float dot_f32_scalar(const float *a, const float *b, size_t len) {
    /* simd.rs:24-45 */
    size_t chunks = len / 4;
    float acc0 = 0.0f, acc1 = 0.0f, acc2 = 0.0f, acc3 = 0.0f;
    for (size_t i = 0; i < chunks; ++i) {
        size_t base = i * 4;
        acc0 += a[base] * b[base];
        acc1 += a[base + 1] * b[base + 1];
        acc2 += a[base + 2] * b[base + 2];
        acc3 += a[base + 3] * b[base + 3];
    }
    float sum = (acc0 + acc1) + (acc2 + acc3);
    for (size_t i = chunks * 4; i < len; ++i) sum += a[i] * b[i];
    return sum;
}

#if WRS_HAVE_X86
__attribute__((target("avx2,fma"))) static float hsum256(__m256 acc) {
    /* simd.rs:108-119, attention.rs:278-288 (identical bodies) */
    __m128 hi_128 = _mm256_extractf128_ps(acc, 1);
    __m128 lo_128 = _mm256_castps256_ps128(acc);
    __m128 sum128 = _mm_add_ps(lo_128, hi_128);
    __m128 shuf = _mm_movehl_ps(sum128, sum128);
    __m128 sum64 = _mm_add_ps(sum128, shuf);
    __m128 shuf2 = _mm_shuffle_ps(sum64, sum64, 1);
    __m128 sum32 = _mm_add_ss(sum64, shuf2);
    return _mm_cvtss_f32(sum32);
}

__attribute__((target("avx2,fma"))) static float dot_f32_avx2(const float *a,
                                                              const float *b,
                                                              size_t len) {
    /* simd.rs:49-106 */
    const float *p_a = a, *p_b = b;
    __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
    __m256 acc2 = _mm256_setzero_ps(), acc3 = _mm256_setzero_ps();
    size_t n_blocks = len / 32;
    for (size_t i = 0; i < n_blocks; ++i) {
        acc0 = _mm256_fmadd_ps(_mm256_loadu_ps(p_a), _mm256_loadu_ps(p_b), acc0);
        acc1 = _mm256_fmadd_ps(_mm256_loadu_ps(p_a + 8), _mm256_loadu_ps(p_b + 8), acc1);
        acc2 = _mm256_fmadd_ps(_mm256_loadu_ps(p_a + 16), _mm256_loadu_ps(p_b + 16), acc2);
        acc3 = _mm256_fmadd_ps(_mm256_loadu_ps(p_a + 24), _mm256_loadu_ps(p_b + 24), acc3);
        p_a += 32;
        p_b += 32;
    }
    __m256 acc01 = _mm256_add_ps(acc0, acc1);
    __m256 acc23 = _mm256_add_ps(acc2, acc3);
    __m256 acc = _mm256_add_ps(acc01, acc23);
    size_t remaining_chunks = (len % 32) / 8;
    for (size_t i = 0; i < remaining_chunks; ++i) {
        acc = _mm256_fmadd_ps(_mm256_loadu_ps(p_a), _mm256_loadu_ps(p_b), acc);
        p_a += 8;
        p_b += 8;
    }
    float result = hsum256(acc);
    size_t tail_offset = len - (len % 8);
    for (size_t i = tail_offset; i < len; ++i) result += a[i] * b[i];
    return result;
}
#endif

float wrs_oracle_dot_f32(const float *a, const float *b, size_t n) {
#if WRS_HAVE_X86
    if (wrs_oracle_uses_avx2()) return dot_f32_avx2(a, b, n);
#endif
    return dot_f32_scalar(a, b, n);
}

/* ------------------------------------------------------------------------ */
/* attention.rs:246-434 single_token_mha_d64                                 */
/* ------------------------------------------------------------------------ */
static void single_token_scalar(const float *q, const float *k, size_t k_stride,
                                const float *v, size_t v_stride, size_t t_kv,
                                float scale, size_t n_heads, float *out,
                                float *scores) {
    /* attention.rs:393-434 */
    for (size_t h = 0; h < n_heads; ++h) {
        size_t head_offset = h * 64;
        const float *q_h = q + head_offset;
        float *out_h = out + head_offset;
        for (size_t j = 0; j < t_kv; ++j) {
            const float *k_vec = k + j * k_stride + head_offset;
            float dot = 0.0f;
            for (int d = 0; d < 64; ++d) dot += q_h[d] * k_vec[d];
            scores[j] = dot * scale;
        }
        wrs_oracle_softmax_inplace(scores, t_kv);
        for (int d = 0; d < 64; ++d) out_h[d] = 0.0f;
        for (size_t j = 0; j < t_kv; ++j) {
            float w = scores[j];
            if (w < 1e-7f) continue; /* :425 */
            const float *v_vec = v + j * v_stride + head_offset;
            for (int d = 0; d < 64; ++d) out_h[d] += w * v_vec[d];
        }
    }
}

#if WRS_HAVE_X86
__attribute__((target("avx2,fma"))) static void single_token_avx2(
    const float *q, const float *k, size_t k_stride, const float *v,
    size_t v_stride, size_t t_kv, float scale, size_t n_heads, float *out,
    float *scores) {
    /* attention.rs:293-390 */
    __m256 v_scale = _mm256_set1_ps(scale);
    for (size_t h = 0; h < n_heads; ++h) {
        size_t head_offset = h * 64;
        const float *q_ptr = q + head_offset;
        const float *k_head_ptr = k + head_offset;
        const float *v_head_ptr = v + head_offset;
        float *out_head_ptr = out + head_offset;
        /* q pre-scaled by 0.125 (:329-336) */
        __m256 vq0 = _mm256_mul_ps(_mm256_loadu_ps(q_ptr), v_scale);
        __m256 vq1 = _mm256_mul_ps(_mm256_loadu_ps(q_ptr + 8), v_scale);
        __m256 vq2 = _mm256_mul_ps(_mm256_loadu_ps(q_ptr + 16), v_scale);
        __m256 vq3 = _mm256_mul_ps(_mm256_loadu_ps(q_ptr + 24), v_scale);
        __m256 vq4 = _mm256_mul_ps(_mm256_loadu_ps(q_ptr + 32), v_scale);
        __m256 vq5 = _mm256_mul_ps(_mm256_loadu_ps(q_ptr + 40), v_scale);
        __m256 vq6 = _mm256_mul_ps(_mm256_loadu_ps(q_ptr + 48), v_scale);
        __m256 vq7 = _mm256_mul_ps(_mm256_loadu_ps(q_ptr + 56), v_scale);
        for (size_t j = 0; j < t_kv; ++j) {
            /* two-accumulator dot order, :338-351 */
            const float *kj = k_head_ptr + j * k_stride;
            __m256 dot0 = _mm256_mul_ps(vq0, _mm256_loadu_ps(kj));
            __m256 dot1 = _mm256_mul_ps(vq1, _mm256_loadu_ps(kj + 8));
            dot0 = _mm256_fmadd_ps(vq2, _mm256_loadu_ps(kj + 16), dot0);
            dot1 = _mm256_fmadd_ps(vq3, _mm256_loadu_ps(kj + 24), dot1);
            dot0 = _mm256_fmadd_ps(vq4, _mm256_loadu_ps(kj + 32), dot0);
            dot1 = _mm256_fmadd_ps(vq5, _mm256_loadu_ps(kj + 40), dot1);
            dot0 = _mm256_fmadd_ps(vq6, _mm256_loadu_ps(kj + 48), dot0);
            dot1 = _mm256_fmadd_ps(vq7, _mm256_loadu_ps(kj + 56), dot1);
            scores[j] = hsum256(_mm256_add_ps(dot0, dot1));
        }
        wrs_oracle_softmax_inplace(scores, t_kv);
        __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
        __m256 acc2 = _mm256_setzero_ps(), acc3 = _mm256_setzero_ps();
        __m256 acc4 = _mm256_setzero_ps(), acc5 = _mm256_setzero_ps();
        __m256 acc6 = _mm256_setzero_ps(), acc7 = _mm256_setzero_ps();
        for (size_t j = 0; j < t_kv; ++j) {
            float w = scores[j];
            if (w < 1e-7f) continue; /* :366 */
            __m256 vw = _mm256_set1_ps(w);
            const float *vj = v_head_ptr + j * v_stride;
            acc0 = _mm256_fmadd_ps(vw, _mm256_loadu_ps(vj), acc0);
            acc1 = _mm256_fmadd_ps(vw, _mm256_loadu_ps(vj + 8), acc1);
            acc2 = _mm256_fmadd_ps(vw, _mm256_loadu_ps(vj + 16), acc2);
            acc3 = _mm256_fmadd_ps(vw, _mm256_loadu_ps(vj + 24), acc3);
            acc4 = _mm256_fmadd_ps(vw, _mm256_loadu_ps(vj + 32), acc4);
            acc5 = _mm256_fmadd_ps(vw, _mm256_loadu_ps(vj + 40), acc5);
            acc6 = _mm256_fmadd_ps(vw, _mm256_loadu_ps(vj + 48), acc6);
            acc7 = _mm256_fmadd_ps(vw, _mm256_loadu_ps(vj + 56), acc7);
        }
        _mm256_storeu_ps(out_head_ptr, acc0);
        _mm256_storeu_ps(out_head_ptr + 8, acc1);
        _mm256_storeu_ps(out_head_ptr + 16, acc2);
        _mm256_storeu_ps(out_head_ptr + 24, acc3);
        _mm256_storeu_ps(out_head_ptr + 32, acc4);
        _mm256_storeu_ps(out_head_ptr + 40, acc5);
        _mm256_storeu_ps(out_head_ptr + 48, acc6);
        _mm256_storeu_ps(out_head_ptr + 56, acc7);
    }
}
#endif

int wrs_oracle_single_token_mha_d64(const float *q, const float *k,
                                    const float *v, size_t t_kv,
                                    size_t n_heads, size_t d_model, float *out) {
    /* The reference indexes head h at h*64 of every row without an assert;
     * a head past the row end would panic (scalar) or read out of bounds. */
    if (n_heads * 64 > d_model) return -3;
    const float scale = 0.125f; /* :255 */
    /* scores buffer: stack of 1500, heap above (:307-314); one buffer reused
     * across heads in both bodies. */
    float stack_buf[1500];
    float *scores = stack_buf;
    if (t_kv > 1500) {
        scores = (float *)malloc(t_kv * sizeof(float));
        if (!scores) return -12;
    }
#if WRS_HAVE_X86
    if (wrs_oracle_uses_avx2())
        single_token_avx2(q, k, d_model, v, d_model, t_kv, scale, n_heads, out,
                          scores);
    else
#endif
        single_token_scalar(q, k, d_model, v, d_model, t_kv, scale, n_heads,
                            out, scores);
    if (scores != stack_buf) free(scores);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* attention.rs:68-243 flash_attention_2                                     */
/* ------------------------------------------------------------------------ */

/* C[m x n] = alpha * A[m x kd] * B[kd x n] + beta * C, each C element a
 * sequential FMA chain over the contraction index starting from zero (the
 * matrixmultiply micro-kernel's order), alpha/beta applied afterwards. B is
 * given packed as Bp[p * n + j]. beta is 0 (overwrite) or 1 (accumulate),
 * the only two values attention.rs passes. */
__attribute__((target_clones("arch=haswell", "default"))) static void
sgemm_tile(size_t m, size_t kd, size_t n, float alpha, const float *a,
           size_t rsa, const float *bp, int accumulate, float *c, size_t rsc,
           float *ab) {
    for (size_t i = 0; i < m; ++i) {
        for (size_t j = 0; j < n; ++j) ab[j] = 0.0f;
        const float *ai = a + i * rsa;
        for (size_t p = 0; p < kd; ++p) {
            float av = ai[p];
            const float *bpp = bp + p * n;
            for (size_t j = 0; j < n; ++j) ab[j] = fmaf(av, bpp[j], ab[j]);
        }
        float *ci = c + i * rsc;
        if (accumulate) {
            for (size_t j = 0; j < n; ++j) ci[j] = alpha * ab[j] + ci[j];
        } else {
            for (size_t j = 0; j < n; ++j) ci[j] = alpha * ab[j];
        }
    }
}

static void fa2_task(const float *q, const float *k, const float *v, size_t t_q,
                     size_t t_kv, size_t d_model, size_t d_head, int causal,
                     float scale, size_t task, size_t n_q_tiles, float *out,
                     float *work) {
    const size_t QT = WRS_ORACLE_Q_TILE, KT = WRS_ORACLE_KV_TILE;
    size_t h = task / n_q_tiles;                  /* :112 */
    size_t i0 = (task % n_q_tiles) * QT;          /* :113 */
    size_t tr = (t_q - i0) < QT ? (t_q - i0) : QT; /* :114 */
    size_t head_offset = h * d_head;

    float *scores = work;                  /* tr * KV_TILE (:120) */
    float *acc = scores + QT * KT;         /* tr * d_head  (:121) */
    float *packed = acc + QT * d_head;     /* packed K^T tile or V tile */
    float *ab = packed + KT * d_head;      /* one row of micro-kernel sums */
    float row_max[WRS_ORACLE_Q_TILE], row_sum[WRS_ORACLE_Q_TILE];
    memset(scores, 0, sizeof(float) * tr * KT);
    memset(acc, 0, sizeof(float) * tr * d_head);
    for (size_t r = 0; r < QT; ++r) {
        row_max[r] = -INFINITY;
        row_sum[r] = 0.0f;
    }
    const float *p_q = q + i0 * d_model + head_offset;

    for (size_t j0 = 0; j0 < t_kv; j0 += KT) {
        if (causal && j0 > i0 + tr - 1) break; /* :132-134 */
        size_t tc = (t_kv - j0) < KT ? (t_kv - j0) : KT;

        /* S = scale * Q_tile K_tile^T, rows of stride KV_TILE (:141-156) */
        for (size_t p = 0; p < d_head; ++p)
            for (size_t c = 0; c < tc; ++c)
                packed[p * tc + c] = k[(j0 + c) * d_model + head_offset + p];
        sgemm_tile(tr, d_head, tc, scale, p_q, d_model, packed, 0, scores, KT, ab);

        for (size_t r = 0; r < tr; ++r) { /* :159-202 */
            float *row = scores + r * KT;
            size_t end = tc;
            if (causal) {
                size_t lim = i0 + r + 1;
                end = lim > j0 ? lim - j0 : 0;
                if (end > tc) end = tc;
            }
            if (end == 0) {
                for (size_t c = 0; c < tc; ++c) row[c] = 0.0f;
                continue;
            }
            float m_tile = -INFINITY;
            for (size_t c = 0; c < end; ++c) m_tile = fmaxf(m_tile, row[c]);
            float m_prev = row_max[r];
            float m_new = fmaxf(m_prev, m_tile);
            float alpha = (m_prev == -INFINITY) ? 0.0f : expf(m_prev - m_new);
            float l_tile = 0.0f;
            for (size_t c = 0; c < end; ++c) {
                float p = expf(row[c] - m_new);
                row[c] = p;
                l_tile += p;
            }
            for (size_t c = end; c < tc; ++c) row[c] = 0.0f; /* :192 */
            row_max[r] = m_new;
            row_sum[r] = row_sum[r] * alpha + l_tile;
            if (alpha != 1.0f) {
                float *acc_row = acc + r * d_head;
                for (size_t d = 0; d < d_head; ++d) acc_row[d] *= alpha;
            }
        }

        /* acc += P_tile V_tile (:207-222) */
        for (size_t c = 0; c < tc; ++c)
            memcpy(packed + c * d_head, v + (j0 + c) * d_model + head_offset,
                   sizeof(float) * d_head);
        sgemm_tile(tr, tc, d_head, 1.0f, scores, KT, packed, 1, acc, d_head, ab);
    }

    for (size_t r = 0; r < tr; ++r) { /* :228-241 */
        float inv_sum = row_sum[r] > 0.0f ? 1.0f / row_sum[r] : 0.0f;
        float *dst = out + (i0 + r) * d_model + head_offset;
        const float *acc_row = acc + r * d_head;
        for (size_t d = 0; d < d_head; ++d) dst[d] = acc_row[d] * inv_sum;
    }
}

int wrs_oracle_flash_attention_2(const float *q, const float *k, const float *v,
                                 size_t t_q, size_t t_kv, size_t n_heads,
                                 size_t d_model, int causal, float *out,
                                 int n_threads) {
    if (n_heads == 0) return -1;           /* :79 */
    if (d_model % n_heads != 0) return -2; /* :80-83 */
    size_t d_head = d_model / n_heads;
    if (t_q == 0) return 0; /* :90-92 */
    if (t_kv == 0) {        /* :93-96 */
        memset(out, 0, sizeof(float) * t_q * d_model);
        return 0;
    }
    if (t_q == 1 && d_head == 64 && !causal) /* :102-105 */
        return wrs_oracle_single_token_mha_d64(q, k, v, t_kv, n_heads, d_model,
                                               out);

    const float scale = 1.0f / sqrtf((float)d_head); /* :107 */
    const size_t QT = WRS_ORACLE_Q_TILE, KT = WRS_ORACLE_KV_TILE;
    size_t n_q_tiles = (t_q + QT - 1) / QT;
    size_t n_tasks = n_heads * n_q_tiles;
    size_t work_floats = QT * KT + QT * d_head + KT * d_head +
                         (KT > d_head ? KT : d_head);
    int err = 0;
#ifdef _OPENMP
    int nt = n_threads > 0 ? n_threads : omp_get_num_procs();
#pragma omp parallel num_threads(nt)
#endif
    {
        float *work = (float *)malloc(sizeof(float) * work_floats);
        if (!work) {
#ifdef _OPENMP
#pragma omp atomic write
#endif
            err = -12;
        } else {
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
            for (size_t task = 0; task < n_tasks; ++task)
                fa2_task(q, k, v, t_q, t_kv, d_model, d_head, causal, scale, task,
                         n_q_tiles, out, work);
            free(work);
        }
    }
    (void)n_threads;
    return err;
}

int wrs_oracle_multi_head_attention(const float *q, const float *k,
                                    const float *v, size_t t_q, size_t t_kv,
                                    size_t n_heads, size_t d_model, int causal,
                                    float *out, int n_threads) {
    /* attention.rs:29-41 */
    return wrs_oracle_flash_attention_2(q, k, v, t_q, t_kv, n_heads, d_model,
                                        causal, out, n_threads);
}

/* ------------------------------------------------------------------------ */
/* crates/tensor/tests/bench_flash_attention_tiled.rs:46-107                 */
/* materialized_attention: the implementation the tiled kernel replaced and  */
/* the reference's own timing baseline. Per head (parallel over heads, as    */
/* into_par_iter): S = scale * (Q K^T) into a t_q x t_kv buffer (sgemm with   */
/* alpha = scale: the dot product, then the scale), softmax_inplace per row,  */
/* then O = S V. No causal mask, no t_kv == 0 special case (the benchmark    */
/* shapes have neither).                                                     */
/* ------------------------------------------------------------------------ */
int wrs_oracle_materialized_attention(const float *q, const float *k, const float *v,
                                      size_t t_q, size_t t_kv, size_t n_heads,
                                      size_t d_model, float *out, int n_threads) {
    if (n_heads == 0 || d_model % n_heads != 0) return -1;
    const size_t d_head = d_model / n_heads;
    const float scale = 1.0f / sqrtf((float)d_head);
    int err = 0;
#ifdef _OPENMP
    int nt = n_threads > 0 ? n_threads : omp_get_num_procs();
#pragma omp parallel for num_threads(nt) schedule(dynamic, 1)
#endif
    for (size_t h = 0; h < n_heads; ++h) {
        const size_t ho = h * d_head;
        float *scores = (float *)malloc(sizeof(float) * (t_q > 0 && t_kv > 0 ? t_q * t_kv : 1));
        if (!scores) {
#ifdef _OPENMP
#pragma omp atomic write
#endif
            err = -12;
            continue;
        }
        for (size_t i = 0; i < t_q; ++i) {
            const float *qi = q + i * d_model + ho;
            for (size_t j = 0; j < t_kv; ++j) {
                const float *kj = k + j * d_model + ho;
                float acc = 0.0f;
                for (size_t d = 0; d < d_head; ++d) acc = fmaf(qi[d], kj[d], acc);
                scores[i * t_kv + j] = scale * acc;
            }
            wrs_oracle_softmax_inplace(scores + i * t_kv, t_kv);
        }
        for (size_t i = 0; i < t_q; ++i) {
            float *oi = out + i * d_model + ho;
            for (size_t d = 0; d < d_head; ++d) oi[d] = 0.0f;
            for (size_t j = 0; j < t_kv; ++j) {
                const float w = scores[i * t_kv + j];
                const float *vj = v + j * d_model + ho;
                for (size_t d = 0; d < d_head; ++d) oi[d] = fmaf(w, vj[d], oi[d]);
            }
        }
        free(scores);
    }
    return err;
}

/* ------------------------------------------------------------------------ */
/* decoder.rs:835-892 multi_head_attention_with_cache                        */
/* ------------------------------------------------------------------------ */
int wrs_oracle_mha_with_cache(const float *q, const float *k, const float *v,
                              size_t n_tokens, size_t total_tokens,
                              size_t t_past, size_t n_heads, size_t d_model,
                              float *out) {
    if (n_heads == 0) return -1;
    if (d_model % n_heads != 0) return -2;
    /* Query i may see keys 0..=t_past+i; the score buffer has total_tokens
     * entries, so the reference panics past that. */
    if (n_tokens > 0 && t_past + n_tokens > total_tokens) return -4;
    size_t d_head = d_model / n_heads;
    if (n_tokens == 1 && d_head == 64) /* :852-855 */
        return wrs_oracle_single_token_mha_d64(q, k, v, t_past + 1, n_heads,
                                               d_model, out);
    const float scale = 1.0f / sqrtf((float)d_head);
    float *scores = (float *)malloc(sizeof(float) * (total_tokens ? total_tokens : 1));
    if (!scores) return -12;
    for (size_t h = 0; h < n_heads; ++h) {
        size_t head_offset = h * d_head;
        for (size_t i = 0; i < n_tokens; ++i) {
            const float *q_vec = q + i * d_model + head_offset;
            size_t max_j = t_past + i + 1;
            for (size_t j = 0; j < max_j; ++j)
                scores[j] = wrs_oracle_dot_f32(q_vec, k + j * d_model + head_offset,
                                               d_head) * scale;
            wrs_oracle_softmax_inplace(scores, max_j);
            float *out_vec = out + i * d_model + head_offset;
            for (size_t d = 0; d < d_head; ++d) out_vec[d] = 0.0f;
            for (size_t j = 0; j < max_j; ++j) {
                float w = scores[j];
                if (w < 1e-7f) continue; /* :884 */
                const float *v_vec = v + j * d_model + head_offset;
                for (size_t d = 0; d < d_head; ++d) out_vec[d] += w * v_vec[d];
            }
        }
    }
    free(scores);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* simd.rs:593-700 dot_f16_f32, quant.rs:343-473 f16_linear                  */
/* ------------------------------------------------------------------------ */
/* IEEE binary16 -> binary32, exact (half::f16::to_f32 / vcvtph2ps). */
static float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0x1Fu) {
        bits = sign | 0x7F800000u | (man << 13);
    } else if (exp != 0) {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    } else if (man == 0) {
        bits = sign;
    } else { /* subnormal: normalize */
        int e = -1;
        do { man <<= 1; ++e; } while (!(man & 0x400u));
        bits = sign | ((uint32_t)(112 - e) << 23) | ((man & 0x3FFu) << 13);
    }
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

float wrs_oracle_f16_to_f32(uint16_t h) { return f16_to_f32(h); }

static float dot_f16_f32_scalar(const uint16_t *w, const float *x, size_t len) {
    /* simd.rs:614-639 */
    float acc0 = 0.0f, acc1 = 0.0f, acc2 = 0.0f, acc3 = 0.0f;
    size_t i = 0;
    while (i + 4 <= len) {
        acc0 += f16_to_f32(w[i]) * x[i];
        acc1 += f16_to_f32(w[i + 1]) * x[i + 1];
        acc2 += f16_to_f32(w[i + 2]) * x[i + 2];
        acc3 += f16_to_f32(w[i + 3]) * x[i + 3];
        i += 4;
    }
    float sum = (acc0 + acc1) + (acc2 + acc3);
    for (; i < len; ++i) sum += f16_to_f32(w[i]) * x[i];
    return sum;
}

#if WRS_HAVE_X86
__attribute__((target("avx2,fma,f16c"))) static float dot_f16_f32_avx2(const uint16_t *w,
                                                                       const float *x,
                                                                       size_t len) {
    /* simd.rs:641-700: four accumulators over 32-element blocks, their sum,
     * then 8-element chunks, hsum, scalar tail. */
    __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
    __m256 acc2 = _mm256_setzero_ps(), acc3 = _mm256_setzero_ps();
    size_t n_blocks = len / 32;
    for (size_t b = 0; b < n_blocks; ++b) {
        const uint16_t *pw = w + b * 32;
        const float *px = x + b * 32;
        acc0 = _mm256_fmadd_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)pw)),
                               _mm256_loadu_ps(px), acc0);
        acc1 = _mm256_fmadd_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(pw + 8))),
                               _mm256_loadu_ps(px + 8), acc1);
        acc2 = _mm256_fmadd_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(pw + 16))),
                               _mm256_loadu_ps(px + 16), acc2);
        acc3 = _mm256_fmadd_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(pw + 24))),
                               _mm256_loadu_ps(px + 24), acc3);
    }
    __m256 acc = _mm256_add_ps(_mm256_add_ps(acc0, acc1), _mm256_add_ps(acc2, acc3));
    size_t i = n_blocks * 32;
    for (; i + 8 <= len; i += 8)
        acc = _mm256_fmadd_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(w + i))),
                              _mm256_loadu_ps(x + i), acc);
    float result = hsum256(acc);
    for (; i < len; ++i) result += f16_to_f32(w[i]) * x[i];
    return result;
}
#endif

float wrs_oracle_dot_f16_f32(const uint16_t *w, const float *x, size_t len) {
#if WRS_HAVE_X86
    /* simd.rs:596-604: the AVX2 body needs avx2, fma and f16c */
    if (wrs_oracle_uses_avx2() && __builtin_cpu_supports("f16c")) return dot_f16_f32_avx2(w, x, len);
#endif
    return dot_f16_f32_scalar(w, x, len);
}

/* output[t * rows + r] = dot_f16_f32(W[r], x[t]) + bias[r] (quant.rs:415-473;
 * the single-token branch, quant.rs:343-413, computes the same per row). Rows
 * run in parallel with no cross-row reduction, so the result does not depend
 * on the thread count. */
int wrs_oracle_f16_linear(const uint16_t *w, size_t rows, size_t cols, const float *x,
                          const float *bias, size_t num_tokens, float *out, int n_threads) {
    if (num_tokens == 0 || rows == 0 || cols == 0) return 0; /* quant.rs:430-432 */
    int nt = n_threads > 0 ? n_threads : omp_get_num_procs();
#pragma omp parallel for num_threads(nt) schedule(static)
    for (long r = 0; r < (long)rows; ++r) {
        const uint16_t *wr = w + (size_t)r * cols;
        float b = bias ? bias[r] : 0.0f;
        for (size_t t = 0; t < num_tokens; ++t) {
            float dot = wrs_oracle_dot_f16_f32(wr, x + t * cols, cols);
            out[t * rows + (size_t)r] = bias ? dot + b : dot;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* norm.rs:1-143 layer_norm, gelu.rs:1-23 gelu_inplace                       */
/* ------------------------------------------------------------------------ */
static void layer_norm_row_scalar(const float *in, const float *gamma, const float *beta,
                                  float eps, size_t d, float *out) {
    /* norm.rs:67-92 */
    float sum = 0.0f;
    for (size_t i = 0; i < d; ++i) sum += in[i];
    float mean = sum / (float)d;
    float sum_sq = 0.0f;
    for (size_t i = 0; i < d; ++i) {
        float diff = in[i] - mean;
        sum_sq += diff * diff;
    }
    float variance = sum_sq / (float)d;
    float inv_std = 1.0f / sqrtf(variance + eps);
    for (size_t i = 0; i < d; ++i) out[i] = (in[i] - mean) * inv_std * gamma[i] + beta[i];
}

#if WRS_HAVE_X86
__attribute__((target("avx2,fma"))) static void layer_norm_row_avx2(const float *in,
                                                                   const float *gamma,
                                                                   const float *beta, float eps,
                                                                   size_t d, float *out) {
    /* norm.rs:3-64: 8-wide sums, hsum, scalar tails; normalize with fma(norm, g, b) */
    size_t n_blocks = d / 8;
    __m256 acc_sum = _mm256_setzero_ps();
    for (size_t i = 0; i < n_blocks; ++i) acc_sum = _mm256_add_ps(acc_sum, _mm256_loadu_ps(in + 8 * i));
    float sum = hsum256(acc_sum);
    for (size_t i = n_blocks * 8; i < d; ++i) sum += in[i];
    float mean = sum / (float)d;
    __m256 v_mean = _mm256_set1_ps(mean);
    __m256 acc_var = _mm256_setzero_ps();
    for (size_t i = 0; i < n_blocks; ++i) {
        __m256 diff = _mm256_sub_ps(_mm256_loadu_ps(in + 8 * i), v_mean);
        acc_var = _mm256_fmadd_ps(diff, diff, acc_var);
    }
    float sum_sq = hsum256(acc_var);
    for (size_t i = n_blocks * 8; i < d; ++i) {
        float diff = in[i] - mean;
        sum_sq += diff * diff;
    }
    float variance = sum_sq / (float)d;
    float inv_std = 1.0f / sqrtf(variance + eps);
    __m256 v_inv_std = _mm256_set1_ps(inv_std);
    for (size_t i = 0; i < n_blocks; ++i) {
        __m256 diff = _mm256_sub_ps(_mm256_loadu_ps(in + 8 * i), v_mean);
        __m256 norm = _mm256_mul_ps(diff, v_inv_std);
        _mm256_storeu_ps(out + 8 * i, _mm256_fmadd_ps(norm, _mm256_loadu_ps(gamma + 8 * i),
                                                      _mm256_loadu_ps(beta + 8 * i)));
    }
    for (size_t i = n_blocks * 8; i < d; ++i) out[i] = (in[i] - mean) * inv_std * gamma[i] + beta[i];
}
#endif

int wrs_oracle_layer_norm(const float *in, const float *gamma, const float *beta, float eps,
                          size_t num_tokens, size_t d_model, float *out) {
    /* norm.rs:116-143: rows in parallel (no cross-row arithmetic) */
#pragma omp parallel for schedule(static) if (num_tokens > 1)
    for (long t = 0; t < (long)num_tokens; ++t) {
        const float *ri = in + (size_t)t * d_model;
        float *ro = out + (size_t)t * d_model;
#if WRS_HAVE_X86
        if (wrs_oracle_uses_avx2()) {
            layer_norm_row_avx2(ri, gamma, beta, eps, d_model, ro);
            continue;
        }
#endif
        layer_norm_row_scalar(ri, gamma, beta, eps, d_model, ro);
    }
    return 0;
}

/* gelu.rs:3-9: 0.5 x (1 + tanh(sqrt(2/pi) x (1 + 0.044715 x^2))), evaluated in
 * the same order of operations (Rust does not contract a*b+c into an FMA). */
float wrs_oracle_gelu(float x) {
    const float GELU_COEF_A = 0.044715f, SQRT_2_OVER_PI = 0.7978846f;
    float inner = SQRT_2_OVER_PI * x * (1.0f + GELU_COEF_A * x * x);
    return 0.5f * x * (1.0f + tanhf(inner));
}

void wrs_oracle_gelu_inplace(float *data, size_t n) {
#pragma omp parallel for schedule(static) if (n >= 4096)
    for (long i = 0; i < (long)n; ++i) data[i] = wrs_oracle_gelu(data[i]);
}

/* ------------------------------------------------------------------------ */
/* decoder.rs:796-828 capture_cross_attention_heads                          */
/* ------------------------------------------------------------------------ */
/* Softmax cross-attention weights of the selected heads: for row i and pair
 * (slot, head), scores_j = dot_f32(q_i[head], k_j[head]) * scale over the
 * n_audio keys (:815-818), softmax_inplace (:819), copied to
 * out[((row_offset + i) * n_selected + slot) * n_audio ..] (:821-822). */
int wrs_oracle_capture_cross_heads(const float *q, const float *k, size_t n_tokens,
                                   size_t n_audio, size_t n_heads, size_t d_model,
                                   const size_t *slots, const size_t *heads, size_t n_pairs,
                                   size_t n_selected, size_t row_offset, float *out) {
    if (n_heads == 0) return -1;
    if (d_model % n_heads != 0) return -2;
    size_t d_head = d_model / n_heads;
    const float scale = 1.0f / sqrtf((float)d_head); /* :810 */
    float *scores = (float *)malloc(sizeof(float) * (n_audio ? n_audio : 1));
    if (!scores) return -12;
    for (size_t i = 0; i < n_tokens; ++i) {
        for (size_t p = 0; p < n_pairs; ++p) {
            size_t head_offset = heads[p] * d_head;
            const float *q_vec = q + i * d_model + head_offset;
            for (size_t j = 0; j < n_audio; ++j)
                scores[j] = wrs_oracle_dot_f32(q_vec, k + j * d_model + head_offset, d_head) *
                            scale;
            wrs_oracle_softmax_inplace(scores, n_audio);
            float *dst = out + ((row_offset + i) * n_selected + slots[p]) * n_audio;
            memcpy(dst, scores, sizeof(float) * n_audio);
        }
    }
    free(scores);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* test_flash_attention_tiled.rs:15-35                                       */
/* ------------------------------------------------------------------------ */
void wrs_oracle_xorshift_fill(uint32_t *state, float *out, size_t n) {
    uint32_t x = *state;
    for (size_t i = 0; i < n; ++i) {
        x ^= x << 13;
        x ^= x >> 17;
        x ^= x << 5;
        out[i] = ((float)x / (float)UINT32_MAX) * 2.0f - 1.0f;
    }
    *state = x;
}
