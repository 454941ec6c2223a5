/*
 * qlm_oracle.c - CPU oracle (TEST INFRASTRUCTURE ONLY; see qlm_oracle.h).
 *
 * Build: gcc -std=c11 -O2 -fno-fast-math -ffp-contract=off -fopenmp (oracle/Makefile).
 * fmaf() stands wherever the reference uses _mm256_fmadd_ps; every other
 * multiply and add is separate. Arrays of 8 model the 8 fp32 lanes of an
 * AVX2 register; hsum8() is the reference's horizontal reduction
 * (lo+hi, hadd, hadd) = ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7)).
 */
#include "qlm_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static int g_threads = 1;

void orc_set_threads(int n) { g_threads = n > 0 ? n : 1; }

static float hsum8(const float* l) {
    return ((l[0] + l[4]) + (l[1] + l[5])) + ((l[2] + l[6]) + (l[3] + l[7]));
}

/* ---- A2: quantiser (safetensors.cpp:296-391) ----------------------------- */

static int8_t clamp127(int q) { return (int8_t)(q < -127 ? -127 : (q > 127 ? 127 : q)); }

/* One group [k0, k1): max|x|, scale = max/127 (1 if zero), inv = 1/scale;
 * the 8-wide vector part rounds half-to-even (_mm256_round_ps, :373-383), a
 * ragged tail of fewer than 8 uses lround (half away from zero, :385-389). */
static void quant_group(const float* x, int n, int8_t* q, float* s) {
    float m = 0.0f;
    for (int i = 0; i < n; ++i) m = fmaxf(m, fabsf(x[i]));
    const float scale = (m > 0.0f) ? (m / 127.0f) : 1.0f;
    *s = scale;
    const float inv = 1.0f / scale;
    const int nv = (n / 8) * 8;
    for (int i = 0; i < nv; ++i) q[i] = clamp127((int)rintf(x[i] * inv));
    for (int i = nv; i < n; ++i) q[i] = clamp127((int)lroundf(x[i] * inv));
}

static void quant_row(const float* row, int K, int group, int8_t* q, float* s) {
    if (group >= K) {
        quant_group(row, K, q, s);
        return;
    }
    const int nb = (K + group - 1) / group;
    for (int b = 0; b < nb; ++b) {
        const int k0 = b * group;
        const int k1 = k0 + group < K ? k0 + group : K;
        quant_group(row + k0, k1 - k0, q + k0, s + b);
    }
}

void orc_quantize_rows_f32(const float* w, int rows, int K, int group, int8_t* q, float* s) {
    const int nb = group >= K ? 1 : (K + group - 1) / group;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (int r = 0; r < rows; ++r)
        quant_row(w + (size_t)r * K, K, group, q + (size_t)r * K, s + (size_t)r * nb);
}

void orc_quantize_rows_bf16(const uint16_t* w, int rows, int K, int group, int8_t* q, float* s) {
    const int nb = group >= K ? 1 : (K + group - 1) / group;
#pragma omp parallel num_threads(g_threads)
    {
        float* tmp = (float*)malloc((size_t)K * sizeof(float));
#pragma omp for schedule(static)
        for (int r = 0; r < rows; ++r) {
            for (int k = 0; k < K; ++k) {
                uint32_t bits = (uint32_t)w[(size_t)r * K + k] << 16;
                memcpy(&tmp[k], &bits, 4);
            }
            quant_row(tmp, K, group, q + (size_t)r * K, s + (size_t)r * nb);
        }
        free(tmp);
    }
}

/* ---- A3: int8 dot (dot8_avx2_int8, math_ops.cpp:448-494) ------------------
 * Per 32-block: four 8-lane products (mul), block = (p0+p1)+(p2+p3) per
 * lane, total = fma(block, scale, total); hsum8; a ragged K%32 tail is a
 * scalar sum scaled by its own block scale. With a per-row scale (group ==
 * K, no reference counterpart) the blocks are added unscaled and the row
 * scale multiplies the final sum. */
static float dot_q8(const float* a, const int8_t* b, const float* s, int K, int rowscale) {
    float total[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int k = 0, blk = 0;
    for (; k + 32 <= K; k += 32, ++blk) {
        for (int l = 0; l < 8; ++l) {
            const float p0 = a[k + l] * (float)b[k + l];
            const float p1 = a[k + 8 + l] * (float)b[k + 8 + l];
            const float p2 = a[k + 16 + l] * (float)b[k + 16 + l];
            const float p3 = a[k + 24 + l] * (float)b[k + 24 + l];
            const float bs = (p0 + p1) + (p2 + p3);
            total[l] = rowscale ? total[l] + bs : fmaf(bs, s[blk], total[l]);
        }
    }
    float r = hsum8(total);
    if (k < K) {
        float tail = 0.0f;
        for (int kk = k; kk < K; ++kk) tail += a[kk] * (float)b[kk];
        r += rowscale ? tail : tail * s[blk];
    }
    return rowscale ? r * s[0] : r;
}

void orc_matmul_i8(const float* A, int M, int K, const int8_t* q, const float* s, int group,
                   int N, float* C, int ldc) {
    const int rowscale = group >= K;
    const int nb = rowscale ? 1 : (K + 31) / 32;
    for (int m = 0; m < M; ++m) {
#pragma omp parallel for schedule(static) num_threads(g_threads)
        for (int n = 0; n < N; ++n)
            C[(size_t)m * ldc + n] =
                dot_q8(A + (size_t)m * K, q + (size_t)n * K, s + (size_t)n * nb, K, rowscale);
    }
}

/* ---- int4 (Q4_0) weights: st_quantize_row_f32_int4 / _bf16_int4
 * (safetensors.cpp:393-515) and the int4 branch of math::matmul
 * (math_ops.cpp:581-818). Per 32-block: scale = max|x|/8 (1 if zero),
 * inv = 1/scale, q = clamp(round(x*inv), -8, 7) stored as the nibble q+8,
 * two columns per byte, low nibble = even column (:397-455). The 8-wide
 * vector part rounds half-to-even (_mm256_round_ps, :426-435); a ragged
 * block tail (fewer than 8 left) uses lround and packs pairs, with nibble 8
 * (value 0) above an odd K's last column (:438-455). */
static int clamp8(int q) { return q < -8 ? -8 : (q > 7 ? 7 : q); }

static void quant4_row(const float* row, int K, uint8_t* out, float* s) {
    const int nb = (K + 31) / 32;
    for (int b = 0; b < nb; ++b) {
        const int k0 = b * 32, k1 = k0 + 32 < K ? k0 + 32 : K;
        float m = 0.0f;
        for (int k = k0; k < k1; ++k) m = fmaxf(m, fabsf(row[k]));
        const float scale = (m > 0.0f) ? (m / 8.0f) : 1.0f;
        s[b] = scale;
        const float inv = 1.0f / scale;
        const int nv = k0 + ((k1 - k0) / 8) * 8;
        for (int k = k0; k < nv; k += 2) {
            const int q0 = clamp8((int)rintf(row[k] * inv));
            const int q1 = clamp8((int)rintf(row[k + 1] * inv));
            out[k / 2] = (uint8_t)(((q1 + 8) << 4) | ((q0 + 8) & 0x0F));
        }
        for (int k = nv; k < k1; k += 2) {
            const int q0 = clamp8((int)lroundf(row[k] * inv));
            const int n1 = k + 1 < k1 ? clamp8((int)lroundf(row[k + 1] * inv)) + 8 : 8;
            out[k / 2] = (uint8_t)((n1 << 4) | ((q0 + 8) & 0x0F));
        }
    }
}

void orc_quantize_rows_q4_f32(const float* w, int rows, int K, uint8_t* q, float* s) {
    const int nb = (K + 31) / 32, pb = (K + 1) / 2;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (int r = 0; r < rows; ++r)
        quant4_row(w + (size_t)r * K, K, q + (size_t)r * pb, s + (size_t)r * nb);
}

void orc_quantize_rows_q4_bf16(const uint16_t* w, int rows, int K, uint8_t* q, float* s) {
    const int nb = (K + 31) / 32, pb = (K + 1) / 2;
#pragma omp parallel num_threads(g_threads)
    {
        float* tmp = (float*)malloc((size_t)K * sizeof(float));
#pragma omp for schedule(static)
        for (int r = 0; r < rows; ++r) {
            for (int k = 0; k < K; ++k) {
                uint32_t bits = (uint32_t)w[(size_t)r * K + k] << 16;
                memcpy(&tmp[k], &bits, 4);
            }
            quant4_row(tmp, K, q + (size_t)r * pb, s + (size_t)r * nb);
        }
        free(tmp);
    }
}

/* Signed values of packed rows: (nibble - 8), Tensor's int4 contract
 * (tensor.hpp:45-56). */
void orc_unpack_q4(const uint8_t* p, int rows, int K, int8_t* q) {
    const int pb = (K + 1) / 2;
    for (int r = 0; r < rows; ++r)
        for (int k = 0; k < K; ++k)
            q[(size_t)r * K + k] =
                (int8_t)(((p[(size_t)r * pb + k / 2] >> ((k & 1) * 4)) & 0x0F) - 8);
}

/* dot_avx2_int4 / dot8_avx2_int4 (math_ops.cpp:604-700) unpack each block
 * and then run dot_avx2_int8's arithmetic unchanged (four 8-lane products,
 * (p0+p1)+(p2+p3), fma with the block scale, hsum8, scaled scalar tail), so
 * the int4 matmul is the int8 one over the unpacked values. */
void orc_matmul_i4(const float* A, int M, int K, const uint8_t* p, const float* s, int N,
                   float* C, int ldc) {
    const int nb = (K + 31) / 32, pb = (K + 1) / 2;
    for (int m = 0; m < M; ++m) {
#pragma omp parallel num_threads(g_threads)
        {
            int8_t* row = (int8_t*)malloc((size_t)K);
#pragma omp for schedule(static)
            for (int n = 0; n < N; ++n) {
                orc_unpack_q4(p + (size_t)n * pb, 1, K, row);
                C[(size_t)m * ldc + n] = dot_q8(A + (size_t)m * K, row, s + (size_t)n * nb, K, 0);
            }
            free(row);
        }
    }
}

/* ---- native weights (--precision bf16: checkpoint dtype kept) ------------
 * fp32 rows: dot_avx2 (math_ops.cpp:209-240), four 8-lane FMA accumulators
 * over 32-column steps, whole 8-column chunks into the first, then
 * (a0+a1)+(a2+a3), hsum8, and a scalar multiply-add tail.
 * bf16 rows: dot_avx2_bf16 / dot8 / dot4 (:245-400, bit-identical per row),
 * two accumulators over 16-column steps (exact bf16 -> fp32 upcast), whole 8-
 * column chunks into the first, a0+a1, hsum8, scalar tail. */
static float bf16_f(uint16_t b) {
    const uint32_t bits = (uint32_t)b << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static float dot_f32w(const float* a, const float* b, int K) {
    float acc[4][8];
    memset(acc, 0, sizeof(acc));
    int k = 0;
    for (; k + 32 <= K; k += 32)
        for (int c = 0; c < 4; ++c)
            for (int l = 0; l < 8; ++l)
                acc[c][l] = fmaf(a[k + 8 * c + l], b[k + 8 * c + l], acc[c][l]);
    for (; k + 8 <= K; k += 8)
        for (int l = 0; l < 8; ++l) acc[0][l] = fmaf(a[k + l], b[k + l], acc[0][l]);
    float s[8];
    for (int l = 0; l < 8; ++l) s[l] = (acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l]);
    float r = hsum8(s);
    for (; k < K; ++k) r += a[k] * b[k];
    return r;
}

static float dot_bf16w(const float* a, const uint16_t* b, int K) {
    float lo[8], hi[8];
    memset(lo, 0, sizeof(lo));
    memset(hi, 0, sizeof(hi));
    int k = 0;
    for (; k + 16 <= K; k += 16)
        for (int l = 0; l < 8; ++l) {
            lo[l] = fmaf(a[k + l], bf16_f(b[k + l]), lo[l]);
            hi[l] = fmaf(a[k + 8 + l], bf16_f(b[k + 8 + l]), hi[l]);
        }
    for (; k + 8 <= K; k += 8)
        for (int l = 0; l < 8; ++l) lo[l] = fmaf(a[k + l], bf16_f(b[k + l]), lo[l]);
    float s[8];
    for (int l = 0; l < 8; ++l) s[l] = lo[l] + hi[l];
    float r = hsum8(s);
    for (; k < K; ++k) r += a[k] * bf16_f(b[k]);
    return r;
}

/* C[m, n] = dot(A[m], W[n]); W fp32 (bf16 = 0) or bf16 bits (bf16 = 1). */
void orc_matmul_w(const float* A, int M, int K, const void* W, int bf16, int N, float* C,
                  int ldc) {
    for (int m = 0; m < M; ++m) {
#pragma omp parallel for schedule(static) num_threads(g_threads)
        for (int n = 0; n < N; ++n)
            C[(size_t)m * ldc + n] =
                bf16 ? dot_bf16w(A + (size_t)m * K, (const uint16_t*)W + (size_t)n * K, K)
                     : dot_f32w(A + (size_t)m * K, (const float*)W + (size_t)n * K, K);
    }
}

/* ---- A5/A6: norms (math_ops.cpp:990-1072, :1133-1172) --------------------- */

float orc_sumsq(const float* x, int n) {
    float a[4][8];
    memset(a, 0, sizeof(a));
    int i = 0;
    const int limit = n - (n % 32);
    for (; i < limit; i += 32)
        for (int j = 0; j < 4; ++j)
            for (int l = 0; l < 8; ++l) {
                const float v = x[i + 8 * j + l];
                a[j][l] = fmaf(v, v, a[j][l]);
            }
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; ++l) a[0][l] = fmaf(x[i + l], x[i + l], a[0][l]);
    float sum[8];
    for (int l = 0; l < 8; ++l) sum[l] = (a[0][l] + a[1][l]) + (a[2][l] + a[3][l]);
    float r = hsum8(sum);
    for (; i < n; ++i) r += x[i] * x[i];
    return r;
}

static void norm_apply_zc(const float* in, const float* w, float* out, float s, int n) {
    for (int i = 0; i < n; ++i) out[i] = (in[i] * s) * (1.0f + w[i]);
}

static void norm_apply_gain(const float* in, const float* w, float* out, float s, int n) {
    for (int i = 0; i < n; ++i) out[i] = (in[i] * s) * w[i];
}

void orc_rms_norm(const float* x, const float* w, float* y, int rows, int n, float eps) {
    for (int r = 0; r < rows; ++r) {
        const float ss = orc_sumsq(x + (size_t)r * n, n);
        const float s = 1.0f / sqrtf((ss / (float)n) + eps);
        norm_apply_zc(x + (size_t)r * n, w, y + (size_t)r * n, s, n);
    }
}

void orc_add_rms_norm(float* res, const float* d, const float* w, float* y, int rows, int n,
                      float eps) {
    for (int r = 0; r < rows; ++r) {
        float* rr = res + (size_t)r * n;
        const float* dr = d + (size_t)r * n;
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        int i = 0;
        for (; i + 8 <= n; i += 8)
            for (int l = 0; l < 8; ++l) {
                const float v = rr[i + l] + dr[i + l];
                rr[i + l] = v;
                acc[l] = fmaf(v, v, acc[l]);
            }
        float ss = hsum8(acc);
        for (; i < n; ++i) {
            const float v = rr[i] + dr[i];
            rr[i] = v;
            ss += v * v;
        }
        const float s = 1.0f / sqrtf((ss / (float)n) + eps);
        norm_apply_zc(rr, w, y + (size_t)r * n, s, n);
    }
}

/* ---- A7 (math_ops.cpp:1076-1129) ------------------------------------------ */

static float silu1(float x) { return x / (1.0f + expf(-x)); }

void orc_silu_mul(float* a, const float* b, int n) {
    for (int i = 0; i < n; ++i) a[i] = silu1(a[i]) * b[i];
}

/* ---- A8 RoPE (math_ops.cpp:1237-1289) ------------------------------------- */

void orc_rope_table(float theta, int rot, int n_pos, float* cos_tab, float* sin_tab) {
    const int half = rot / 2;
    for (int p = 0; p < n_pos; ++p)
        for (int i = 0; i < half; ++i) {
            const float inv = 1.0f / powf(theta, (2.0f * (float)i) / (float)rot);
            const float ang = (float)p * inv;
            cos_tab[(size_t)p * half + i] = cosf(ang);
            sin_tab[(size_t)p * half + i] = sinf(ang);
        }
}

void orc_rope_neox(float* t, int num_heads, int head_stride, int pos, float theta, int rot) {
    const int half = rot / 2;
    for (int i = 0; i < half; ++i) {
        const float inv = 1.0f / powf(theta, (2.0f * (float)i) / (float)rot);
        const float ang = (float)pos * inv;
        const float c = cosf(ang), s = sinf(ang);
        for (int h = 0; h < num_heads; ++h) {
            float* hd = t + (size_t)h * head_stride;
            const float x1 = hd[i], x2 = hd[i + half];
            hd[i] = x1 * c - x2 * s;
            hd[i + half] = x2 * c + x1 * s;
        }
    }
}

/* ---- A10 conv (math_ops.cpp:1321-1364) ------------------------------------- */

void orc_conv1d_tapmajor(const float* in, float* state, int oldest, const float* w_t, float* out,
                         int conv_dim, int kernel_size) {
    const int ntaps = kernel_size - 1;
    for (int c = 0; c < conv_dim; ++c) {
        float acc = 0.0f;
        for (int j = 0; j < ntaps; ++j) {
            const int row = (oldest + j) % ntaps;
            acc = acc + state[(size_t)row * conv_dim + c] * w_t[(size_t)j * conv_dim + c];
        }
        acc = acc + in[c] * w_t[(size_t)ntaps * conv_dim + c];
        out[c] = acc;
        state[(size_t)oldest * conv_dim + c] = in[c];
    }
}

/* ---- A12 recurrence (attention.cpp:498-571) -------------------------------- */

static void delta_head(const float* q, const float* k, const float* v, float dec, float beta,
                       float* S, float* out, int d) {
    float* kv = (float*)calloc((size_t)d, sizeof(float));
    float* delta = (float*)malloc((size_t)d * sizeof(float));
    for (int i = 0; i < d; ++i) {
        float* row = S + (size_t)i * d;
        for (int j = 0; j < d; ++j) {
            row[j] = row[j] * dec;
            kv[j] = fmaf(k[i], row[j], kv[j]);
        }
    }
    for (int j = 0; j < d; ++j) delta[j] = v[j] - kv[j];
    for (int i = 0; i < d; ++i) {
        const float s = beta * k[i];
        float* row = S + (size_t)i * d;
        for (int j = 0; j < d; ++j) row[j] = fmaf(s, delta[j], row[j]);
    }
    const float q_scale = 1.0f / sqrtf((float)d);
    for (int j = 0; j < d; ++j) out[j] = 0.0f;
    for (int i = 0; i < d; ++i) {
        const float* row = S + (size_t)i * d;
        for (int j = 0; j < d; ++j) out[j] = fmaf(q[i], row[j], out[j]);
    }
    for (int j = 0; j < d; ++j) out[j] = out[j] * q_scale;
    free(kv);
    free(delta);
}

void orc_gated_delta_step(const float* q, const float* k, const float* v, const float* decay,
                          const float* beta, float* state, float* out, int B, int H, int d) {
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (int bh = 0; bh < B * H; ++bh)
        delta_head(q + (size_t)bh * d, k + (size_t)bh * d, v + (size_t)bh * d, decay[bh], beta[bh],
                   state + (size_t)bh * d * d, out + (size_t)bh * d, d);
}

void orc_deltanet_core(const float* proj, float* conv_state, int oldest, const float* conv_w_t,
                       const float* A_log, const float* dt_bias, const float* norm_w,
                       float* state, float* out, int H, int d) {
    const int HD = H * d;
    const int C = 3 * HD;
    float* x = (float*)malloc((size_t)C * sizeof(float));
    /* conv1d step + SiLU (attention.cpp:441-460) */
    orc_conv1d_tapmajor(proj, conv_state, oldest, conv_w_t, x, C, 4);
    for (int i = 0; i < C; ++i) x[i] = silu1(x[i]);
    float* q = x;
    float* k = x + HD;
    const float* v = x + 2 * HD;
    /* L2 norm per head (:463-470) */
    for (int h = 0; h < H; ++h) {
        float* qh = q + (size_t)h * d;
        float* kh = k + (size_t)h * d;
        const float qn = sqrtf(orc_sumsq(qh, d) + 1e-6f);
        const float kn = sqrtf(orc_sumsq(kh, d) + 1e-6f);
        for (int i = 0; i < d; ++i) qh[i] = qh[i] / qn;
        for (int i = 0; i < d; ++i) kh[i] = kh[i] / kn;
    }
    const float* z = proj + 3 * HD;
    const float* braw = proj + 4 * HD;
    const float* araw = proj + 4 * HD + H;
    for (int h = 0; h < H; ++h) {
        /* gates (:472-483) */
        const float dt_in = araw[h] + dt_bias[h];
        const float sp = (dt_in > 20.0f) ? dt_in : log1pf(expf(dt_in));
        const float alpha = -expf(A_log[h]) * sp;
        const float dec = expf(alpha);
        const float beta = 1.0f / (1.0f + expf(-braw[h]));
        float* oh = out + (size_t)h * d;
        delta_head(q + (size_t)h * d, k + (size_t)h * d, v + (size_t)h * d, dec, beta,
                   state + (size_t)h * d * d, oh, d);
        /* head RMSNorm (:574-578) and SiLU(z) gate (:582-585) */
        const float s = 1.0f / sqrtf((orc_sumsq(oh, d) / (float)d) + 1e-6f);
        norm_apply_gain(oh, norm_w, oh, s, d);
        for (int j = 0; j < d; ++j) {
            const float zv = z[(size_t)h * d + j];
            oh[j] = oh[j] * (zv / (1.0f + expf(-zv)));
        }
    }
    free(x);
}

/* ---- A9 attention (attention.cpp:17-82) ------------------------------------ */

static float dot_f32(const float* a, const float* b, int n) {
    float a0[8] = {0, 0, 0, 0, 0, 0, 0, 0}, a1[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 16 <= n; i += 16)
        for (int l = 0; l < 8; ++l) {
            a0[l] = fmaf(a[i + l], b[i + l], a0[l]);
            a1[l] = fmaf(a[i + 8 + l], b[i + 8 + l], a1[l]);
        }
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; ++l) a0[l] = fmaf(a[i + l], b[i + l], a0[l]);
    float sum[8];
    for (int l = 0; l < 8; ++l) sum[l] = a0[l] + a1[l];
    float r = hsum8(sum);
    for (; i < n; ++i) r += a[i] * b[i];
    return r;
}

static void attend_head(const float* q, const float* kc, const float* vc, float* out, int pos,
                        int kv_size, int kv_off, int hd, float scale) {
    float* sc = (float*)malloc((size_t)(pos + 1) * sizeof(float));
    for (int p = 0; p <= pos; ++p) sc[p] = dot_f32(q, kc + (size_t)p * kv_size + kv_off, hd) * scale;
    float mx = sc[0];
    for (int p = 1; p <= pos; ++p)
        if (sc[p] > mx) mx = sc[p];
    float sum = 0.0f;
    for (int p = 0; p <= pos; ++p) {
        sc[p] = expf(sc[p] - mx);
        sum += sc[p];
    }
    for (int p = 0; p <= pos; ++p) sc[p] = sc[p] / sum;
    for (int i = 0; i < hd; ++i) out[i] = 0.0f;
    for (int p = 0; p <= pos; ++p) {
        const float* vr = vc + (size_t)p * kv_size + kv_off;
        for (int i = 0; i < hd; ++i) out[i] = fmaf(sc[p], vr[i], out[i]);
    }
    free(sc);
}

void orc_attention(const float* q, const float* k_cache, const float* v_cache, int ctx, float* out,
                   int n_q, int n_kv, int hd) {
    const int group = n_q / n_kv;
    const float scale = 1.0f / sqrtf((float)hd);
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (int h = 0; h < n_q; ++h)
        attend_head(q + (size_t)h * hd, k_cache, v_cache, out + (size_t)h * hd, ctx - 1, n_kv * hd,
                    (h / group) * hd, hd, scale);
}

void orc_gqa_core(float* qkv, const float* q_norm, const float* k_norm, float theta, int rot,
                  float* k_cache, float* v_cache, int max_seq, int pos, float* out, int n_q,
                  int n_kv, int hd, int gated) {
    const int qhd = gated ? 2 * hd : hd;
    float* q = qkv;
    float* k = qkv + (size_t)n_q * qhd;
    const float* v = k + (size_t)n_kv * hd;
    (void)max_seq;
    if (q_norm)
        for (int h = 0; h < n_q; ++h) {
            float* qh = q + (size_t)h * qhd;
            const float s = 1.0f / sqrtf((orc_sumsq(qh, hd) / (float)hd) + 1e-6f);
            norm_apply_zc(qh, q_norm, qh, s, hd);
        }
    if (k_norm)
        for (int h = 0; h < n_kv; ++h) {
            float* kh = k + (size_t)h * hd;
            const float s = 1.0f / sqrtf((orc_sumsq(kh, hd) / (float)hd) + 1e-6f);
            norm_apply_zc(kh, k_norm, kh, s, hd);
        }
    orc_rope_neox(k, n_kv, hd, pos, theta, rot);
    for (int h = 0; h < n_q; ++h) orc_rope_neox(q + (size_t)h * qhd, 1, qhd, pos, theta, rot);
    const int kv_size = n_kv * hd;
    memcpy(k_cache + (size_t)pos * kv_size, k, (size_t)kv_size * sizeof(float));
    memcpy(v_cache + (size_t)pos * kv_size, v, (size_t)kv_size * sizeof(float));
    const int group = n_q / n_kv;
    const float scale = 1.0f / sqrtf((float)hd);
    for (int h = 0; h < n_q; ++h)
        attend_head(q + (size_t)h * qhd, k_cache, v_cache, out + (size_t)h * hd, pos, kv_size,
                    (h / group) * hd, hd, scale);
    if (gated)
        for (int h = 0; h < n_q; ++h)
            for (int i = 0; i < hd; ++i) {
                const float g = q[(size_t)h * qhd + hd + i];
                out[(size_t)h * hd + i] = out[(size_t)h * hd + i] * (1.0f / (1.0f + expf(-g)));
            }
}

/* ---- A14 (model.cpp:263-274) ---------------------------------------------- */

int orc_argmax(const float* x, int n) {
    int best = 0;
    float mx = x[0];
    for (int i = 1; i < n; ++i)
        if (x[i] > mx) {
            mx = x[i];
            best = i;
        }
    return best;
}
