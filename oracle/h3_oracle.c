/* CPU oracle of the DiT denoiser path - TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, on the CPU, the arithmetic of the reference engine's
 * bit-exact hand kernels (0xSufi/h3.c, CUDA backend) so that the HIP backend
 * can be checked against it on identical inputs.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * only as the checker: nothing in the product path calls it.
 *
 * Arithmetic contract (reference h3_cuda_internal.h:244-253): bf16 values are
 * widened exactly to f32, every op accumulates in f32, every op output is
 * rounded to bf16 with round-to-nearest-even.  Dot products are sequential
 * fmaf chains (the reference hand kernels' order).  Row statistics (sums of
 * squares, means) are summed in double: the reference's GPU kernels reduce
 * in f32 tree order and its tests accept one bf16 ulp for that
 * (tests/test_cuda_dit.c:57-71); a double sum sits closer to the exact value
 * than any f32 order, so the tests' bound only has to cover the device's
 * own f32 reduction error.
 *
 * Build: oracle/Makefile (gcc -O3 -fopenmp; FMA contraction on so that
 * fmaf-written accumulations stay fused).  Every function cites the
 * reference lines it follows; the pins that check each one are listed in
 * tests/test_oracle_pins.py.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef uint16_t bf16;

static inline float b2f(bf16 v) {
    uint32_t bits = (uint32_t)v << 16;
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

/* RNE narrowing, reference h3_cuda_internal.h:249-253 */
static inline bf16 f2b(float v) {
    uint32_t bits;
    memcpy(&bits, &v, 4);
    if ((bits & 0x7fffffffu) > 0x7f800000u) return (bf16)((bits >> 16) | 0x40);
    bits += 0x7fffu + ((bits >> 16) & 1u);
    return (bf16)(bits >> 16);
}

static inline float rbf(float v) { return b2f(f2b(v)); }

void orc_f32_to_bf16(const float *in, bf16 *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = f2b(in[i]);
}

void orc_bf16_to_f32(const bf16 *in, float *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = b2f(in[i]);
}

/* ------------------------------------------------------------- linear */

/* C[m,n] = bf16(bias[n] + sum_k x[m,k] * w[n,k]) with the sum accumulated
 * by fmaf in increasing k starting from the bias: the reference's hand GEMM
 * h3k_linear_bf16 (h3_cuda_core.cu:358-371), bit for bit.  The loops are
 * blocked (columns x rows) with k innermost-sequential per output so the
 * order of every accumulation is unchanged. */
/* F32 linear, reference h3_cuda_core.cu:343-356 (h3k_linear_f32: one
 * output per thread, fmaf over k from the bias). */
void orc_linear_f32(const float *x, const float *w, const float *bias,
                    float *out, size_t m, size_t k, size_t n) {
#pragma omp parallel for schedule(static) collapse(2)
    for (size_t i = 0; i < m; i++)
        for (size_t j = 0; j < n; j++) {
            float sum = bias ? bias[j] : 0.0f;
            const float *xr = x + i * k, *wr = w + j * k;
            for (size_t kk = 0; kk < k; kk++) sum = fmaf(xr[kk], wr[kk], sum);
            out[i * n + j] = sum;
        }
}

void orc_linear_bf16(const bf16 *x, const bf16 *w, const bf16 *bias,
                     bf16 *out, size_t m, size_t k, size_t n) {
    enum { JB = 64, IB = 4 };
    const size_t col_blocks = (n + JB - 1) / JB;
#pragma omp parallel
    {
        float *wt = (float *)malloc(k * JB * sizeof(float));
        float *xr = (float *)malloc(IB * k * sizeof(float));
#pragma omp for schedule(dynamic)
        for (size_t cb = 0; cb < col_blocks; cb++) {
            const size_t j0 = cb * JB;
            const size_t jn = n - j0 < JB ? n - j0 : JB;
            for (size_t kk = 0; kk < k; kk++)
                for (size_t j = 0; j < JB; j++)
                    wt[kk * JB + j] =
                        j < jn ? b2f(w[(j0 + j) * k + kk]) : 0.0f;
            for (size_t i0 = 0; i0 < m; i0 += IB) {
                const size_t in = m - i0 < IB ? m - i0 : IB;
                for (size_t i = 0; i < in; i++)
                    for (size_t kk = 0; kk < k; kk++)
                        xr[i * k + kk] = b2f(x[(i0 + i) * k + kk]);
                float acc[IB][JB];
                for (size_t i = 0; i < IB; i++)
                    for (size_t j = 0; j < JB; j++)
                        acc[i][j] = bias && j < jn ? b2f(bias[j0 + j]) : 0.0f;
                for (size_t kk = 0; kk < k; kk++) {
                    const float *wk = wt + kk * JB;
                    for (size_t i = 0; i < in; i++) {
                        const float xv = xr[i * k + kk];
                        for (size_t j = 0; j < JB; j++)
                            acc[i][j] = fmaf(xv, wk[j], acc[i][j]);
                    }
                }
                for (size_t i = 0; i < in; i++)
                    for (size_t j = 0; j < jn; j++)
                        out[(i0 + i) * n + j0 + j] = f2b(acc[i][j]);
            }
        }
        free(wt);
        free(xr);
    }
}

/* F32 patch projection into bf16 rows (h3_cuda_core.cu:374-403):
 * out[map ? map[r] : r][j] = bf16(bias[j] + sum_k x[r,k] w[j,k]). */
void orc_patch_linear(const float *x, const float *w, const float *bias,
                      bf16 *out, const uint32_t *map, size_t rows,
                      size_t k, size_t n) {
#pragma omp parallel for schedule(static)
    for (size_t r = 0; r < rows; r++) {
        size_t target = map ? map[r] : r;
        for (size_t j = 0; j < n; j++) {
            float sum = bias ? bias[j] : 0.0f;
            for (size_t kk = 0; kk < k; kk++)
                sum = fmaf(x[r * k + kk], w[j * k + kk], sum);
            out[target * n + j] = f2b(sum);
        }
    }
}

/* ---------------------------------------------------------- row ops */

/* Row statistics: the sum is taken in double (closer to the exact sum than
 * any f32 order; the reference's kernels use an f32 tree, the HIP kernels
 * an f32 wave tree), then the reference's f32 formula
 * 1 / sqrtf(mean + eps) (h3_cuda_dit.cu:160-161). */
static float row_inverse_rms(const float *v, size_t width, float eps) {
    double ss = 0.0;
    for (size_t c = 0; c < width; c++) ss += (double)v[c] * v[c];
    return 1.0f / sqrtf((float)ss / (float)width + eps);
}

/* AdaLN (h3_cuda_dit.cu:141-175):
 * y = bf16(x * inv * w * (1 + mod[scale]) + mod[shift]),
 * mod row = map[r] * slots * width. */
void orc_adaln(const bf16 *x, const bf16 *w, const bf16 *mod,
               const uint32_t *map, bf16 *out, size_t rows, size_t width,
               size_t slots, size_t shift_slot, size_t scale_slot,
               float eps) {
#pragma omp parallel
    {
        float *v = (float *)malloc(width * sizeof(float));
#pragma omp for schedule(static)
        for (size_t r = 0; r < rows; r++) {
            for (size_t c = 0; c < width; c++) v[c] = b2f(x[r * width + c]);
            const float inv = row_inverse_rms(v, width, eps);
            const bf16 *m = mod + (size_t)map[r] * slots * width;
            for (size_t c = 0; c < width; c++) {
                float n = v[c] * inv * b2f(w[c]);
                float shift = b2f(m[shift_slot * width + c]);
                float scale = b2f(m[scale_slot * width + c]);
                out[r * width + c] = f2b(n * (1.0f + scale) + shift);
            }
        }
        free(v);
    }
}

/* Gate (h3_cuda_dit.cu:261-276): y = bf16(res + br * mod[gate]). */
void orc_gate(const bf16 *res, const bf16 *br, const bf16 *mod,
              const uint32_t *map, bf16 *out, size_t rows, size_t width,
              size_t slots, size_t gate_slot) {
#pragma omp parallel for schedule(static)
    for (size_t r = 0; r < rows; r++) {
        const bf16 *m = mod + (size_t)map[r] * slots * width +
                        gate_slot * width;
        for (size_t c = 0; c < width; c++) {
            size_t i = r * width + c;
            out[i] = f2b(b2f(res[i]) + b2f(br[i]) * b2f(m[c]));
        }
    }
}

/* Gate + adaLN (h3_cuda_dit.cu:281-332): the rounded gated row is written
 * out and also normalised. */
void orc_gate_adaln(const bf16 *res, const bf16 *br, const bf16 *w,
                    const bf16 *gate_mod, const bf16 *norm_mod,
                    const uint32_t *map, bf16 *gated, bf16 *out, size_t rows,
                    size_t width, size_t slots, size_t gate_slot,
                    size_t shift_slot, size_t scale_slot, float eps) {
#pragma omp parallel
    {
        float *v = (float *)malloc(width * sizeof(float));
#pragma omp for schedule(static)
        for (size_t r = 0; r < rows; r++) {
            const size_t base = (size_t)map[r] * slots * width;
            for (size_t c = 0; c < width; c++) {
                size_t i = r * width + c;
                bf16 g = f2b(b2f(res[i]) +
                             b2f(br[i]) *
                                 b2f(gate_mod[base + gate_slot * width + c]));
                gated[i] = g;
                v[c] = b2f(g);
            }
            const float inv = row_inverse_rms(v, width, eps);
            for (size_t c = 0; c < width; c++) {
                float n = v[c] * inv * b2f(w[c]);
                float shift = b2f(norm_mod[base + shift_slot * width + c]);
                float scale = b2f(norm_mod[base + scale_slot * width + c]);
                out[r * width + c] = f2b(n * (1.0f + scale) + shift);
            }
        }
        free(v);
    }
}

/* LayerNorm (+ optional affine, h3_cuda_core.cu:250-295) + optional adaLN
 * modulation.  w, b, mod may be NULL. */
void orc_layer_adaln(const bf16 *x, const bf16 *w, const bf16 *b,
                     const bf16 *mod, const uint32_t *map, bf16 *out,
                     size_t rows, size_t width, size_t slots,
                     size_t shift_slot, size_t scale_slot, float eps) {
#pragma omp parallel
    {
        float *v = (float *)malloc(width * sizeof(float));
#pragma omp for schedule(static)
        for (size_t r = 0; r < rows; r++) {
            double sum = 0.0;
            for (size_t c = 0; c < width; c++) {
                v[c] = b2f(x[r * width + c]);
                sum += v[c];
            }
            const float mean = (float)sum / (float)width;
            double sq = 0.0;
            for (size_t c = 0; c < width; c++) {
                double d = (double)(v[c] - mean);
                sq += d * d;
            }
            const float inv = 1.0f / sqrtf((float)sq / (float)width + eps);
            const bf16 *m = mod ? mod + (size_t)map[r] * slots * width : NULL;
            for (size_t c = 0; c < width; c++) {
                float n = (v[c] - mean) * inv;
                if (w && b) n = fmaf(n, b2f(w[c]), b2f(b[c]));
                else if (w) n = n * b2f(w[c]);
                else if (b) n = n + b2f(b[c]);
                if (m)
                    n = n * (1.0f + b2f(m[scale_slot * width + c])) +
                        b2f(m[shift_slot * width + c]);
                out[r * width + c] = f2b(n);
            }
        }
        free(v);
    }
}

/* RMS norm (h3_cuda_core.cu:184-210): y = bf16((x * inv) * w). */
void orc_rms_norm(const bf16 *x, const bf16 *w, bf16 *out, size_t rows,
                  size_t width, float eps) {
#pragma omp parallel
    {
        float *v = (float *)malloc(width * sizeof(float));
#pragma omp for schedule(static)
        for (size_t r = 0; r < rows; r++) {
            for (size_t c = 0; c < width; c++) v[c] = b2f(x[r * width + c]);
            const float inv = row_inverse_rms(v, width, eps);
            for (size_t c = 0; c < width; c++)
                out[r * width + c] = f2b(v[c] * inv * b2f(w[c]));
        }
        free(v);
    }
}

/* In-place per-head RMS norm (h3_cuda_core.cu:322-341). */
void orc_head_rms_norm(bf16 *t, const bf16 *w, size_t rows, size_t heads,
                       size_t hd, float eps) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < rows * heads; i++) {
        bf16 *x = t + i * hd;
        double ss = 0.0;
        for (size_t d = 0; d < hd; d++) ss += (double)b2f(x[d]) * b2f(x[d]);
        const float inv = 1.0f / sqrtf((float)ss / (float)hd + eps);
        for (size_t d = 0; d < hd; d++) x[d] = f2b(b2f(x[d]) * inv * b2f(w[d]));
    }
}

/* Q/K per-head RMS norm + rotate-half RoPE + V copy
 * (h3_cuda_attention.cu:175-237).  grouped: rows [head][q,k,v][hd], else
 * [q,k,v][head][hd]. */
void orc_qkv_rope(const bf16 *qkv, const bf16 *qw, const bf16 *kw,
                  const bf16 *cosines, const bf16 *sines, bf16 *q, bf16 *k,
                  bf16 *v, size_t seq, size_t heads, size_t hd,
                  size_t rope_half, int grouped, float eps) {
    const size_t inner = heads * hd;
#pragma omp parallel
    {
        float *qn = (float *)malloc(hd * sizeof(float));
        float *kn = (float *)malloc(hd * sizeof(float));
#pragma omp for schedule(static)
        for (size_t i = 0; i < seq * heads; i++) {
            const size_t row = i / heads, head = i % heads;
            const size_t rb = row * inner * 3;
            size_t qb = rb + head * hd, kb = qb + inner, vb = qb + 2 * inner;
            if (grouped) {
                qb = rb + head * hd * 3;
                kb = qb + hd;
                vb = kb + hd;
            }
            double qs = 0.0, ks = 0.0;
            for (size_t d = 0; d < hd; d++) {
                double a = b2f(qkv[qb + d]), b = b2f(qkv[kb + d]);
                qs += a * a;
                ks += b * b;
            }
            const float qi = 1.0f / sqrtf((float)qs / (float)hd + eps);
            const float ki = 1.0f / sqrtf((float)ks / (float)hd + eps);
            for (size_t d = 0; d < hd; d++) {
                qn[d] = b2f(qkv[qb + d]) * qi * b2f(qw[d]);
                kn[d] = b2f(qkv[kb + d]) * ki * b2f(kw[d]);
            }
            const size_t ob = (row * heads + head) * hd;
            for (size_t d = 0; d < hd; d++) {
                float q0 = qn[d], k0 = kn[d];
                if (d < rope_half) {
                    float c = b2f(cosines[row * rope_half + d]);
                    float s = b2f(sines[row * rope_half + d]);
                    q0 = qn[d] * c - qn[d + rope_half] * s;
                    k0 = kn[d] * c - kn[d + rope_half] * s;
                } else if (d < 2 * rope_half) {
                    size_t p = d - rope_half;
                    float c = b2f(cosines[row * rope_half + p]);
                    float s = b2f(sines[row * rope_half + p]);
                    q0 = qn[d] * c + qn[p] * s;
                    k0 = kn[d] * c + kn[p] * s;
                }
                q[ob + d] = f2b(q0);
                k[ob + d] = f2b(k0);
                v[ob + d] = qkv[vb + d];
            }
        }
        free(qn);
        free(kn);
    }
}

/* The RoPE pair rotation alone on [rows][heads][hd] bf16 (the rotation
 * step of h3_cuda_attention.cu:218-233, without the Q/K norm): for
 * d < half, x'_d = x_d c - x_{d+half} s and x'_{d+half} = x_{d+half} c +
 * x_d s with c, s = tables[row][d], each as one fused multiply-add over a
 * rounded product, then bf16; dims from 2 half on are copied. */
void orc_rope_rotate(const bf16 *in, const bf16 *cosines, const bf16 *sines,
                     bf16 *out, size_t rows, size_t heads, size_t hd,
                     size_t half) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < rows * heads; i++) {
        const size_t row = i / heads, b = i * hd;
        for (size_t d = 0; d < hd; d++) out[b + d] = in[b + d];
        for (size_t d = 0; d < half && d + half < hd; d++) {
            const float x = b2f(in[b + d]), y = b2f(in[b + d + half]);
            const float c = b2f(cosines[row * half + d]);
            const float s = b2f(sines[row * half + d]);
            const float ys = y * s, xs = x * s;
            out[b + d] = f2b(fmaf(x, c, -ys));
            out[b + d + half] = f2b(fmaf(y, c, xs));
        }
    }
}

/* Non-causal attention, Q [q_rows][heads][hd], K/V [kv_rows][heads][hd].
 * Scores s = scale * sum_d fmaf(q, k) (h3_cuda_attention.cu:505-515);
 * p = exp(s - max).  round_p = 1 applies the flash kernels' rule
 * (h3_cuda_attention.cu:1527-1528, 1780-1787): O = sum bf16(p) v / sum p;
 * round_p = 0 is the naive kernel's sum (p / l) v (:533-546). */
void orc_sdpa(const bf16 *q, const bf16 *k, const bf16 *v, bf16 *out,
              size_t q_rows, size_t kv_rows, size_t heads, size_t hd,
              float scale, int head_major, int round_p) {
    /* One head at a time: its K is widened once into a [hd][kv_rows]
     * transpose and V into [kv_rows][hd], so the score loop runs over keys
     * with d outermost.  Each score is still the sequential fmaf chain over
     * d = 0..hd-1 from 0, so the result does not depend on the layout. */
    const size_t kv = kv_rows ? kv_rows : 1;
    float *kt = (float *)malloc(hd * kv * sizeof(float));
    float *vf = (float *)malloc(kv * hd * sizeof(float));
    for (size_t head = 0; head < heads; head++) {
#pragma omp parallel for schedule(static)
        for (size_t j = 0; j < kv_rows; j++) {
            const bf16 *kr = k + (j * heads + head) * hd;
            const bf16 *vr = v + (j * heads + head) * hd;
            for (size_t d = 0; d < hd; d++) {
                kt[d * kv_rows + j] = b2f(kr[d]);
                vf[j * hd + d] = b2f(vr[d]);
            }
        }
#pragma omp parallel
        {
            float *s = (float *)malloc(kv * sizeof(float));
            float *qf = (float *)malloc(hd * sizeof(float));
            float *acc = (float *)malloc(hd * sizeof(float));
#pragma omp for schedule(dynamic, 4)
            for (size_t row = 0; row < q_rows; row++) {
                const size_t qb = (row * heads + head) * hd;
                for (size_t d = 0; d < hd; d++) qf[d] = b2f(q[qb + d]);
                for (size_t j = 0; j < kv_rows; j++) s[j] = 0.0f;
                for (size_t d = 0; d < hd; d++) {
                    const float qd = qf[d];
                    const float *kd = kt + d * kv_rows;
                    for (size_t j = 0; j < kv_rows; j++)
                        s[j] = fmaf(qd, kd[j], s[j]);
                }
                float mx = -INFINITY;
                for (size_t j = 0; j < kv_rows; j++) {
                    s[j] *= scale;
                    if (s[j] > mx) mx = s[j];
                }
                float l = 0.0f;
                for (size_t j = 0; j < kv_rows; j++) {
                    s[j] = expf(s[j] - mx);
                    l += s[j];
                }
                const float inv = l > 0.0f ? 1.0f / l : 0.0f;
                for (size_t d = 0; d < hd; d++) acc[d] = 0.0f;
                for (size_t j = 0; j < kv_rows; j++) {
                    const float *vr = vf + j * hd;
                    const float p = round_p ? rbf(s[j]) : s[j] * inv;
                    for (size_t d = 0; d < hd; d++)
                        acc[d] = fmaf(p, vr[d], acc[d]);
                }
                const size_t ob = head_major ? (head * q_rows + row) * hd : qb;
                for (size_t d = 0; d < hd; d++)
                    out[ob + d] = f2b(round_p ? acc[d] * inv : acc[d]);
            }
            free(s);
            free(qf);
            free(acc);
        }
    }
    free(kt);
    free(vf);
}

/* Block-sparse joint attention (reference h3_gpu.h:44-52, the FA2 kernel's
 * CSR walk h3_cuda_attention.cu:1652-1673): query row r of block r / 128
 * attends only to the keys of the 64-row tiles listed for its block, with
 * the same softmax as orc_sdpa (max over the kept keys, P rounded to bf16
 * before P.V when round_p).  Lists are clamped to the dense tile count. */
void orc_sdpa_sparse(const bf16 *q, const bf16 *k, const bf16 *v, bf16 *out,
                     size_t rows, size_t heads, size_t hd, float scale,
                     int head_major, int round_p, const uint32_t *ptr,
                     const uint32_t *idx) {
    const size_t tiles = (rows + 63) / 64;
#pragma omp parallel
    {
        float *s = (float *)malloc((rows ? rows : 1) * sizeof(float));
        unsigned char *keep = (unsigned char *)malloc(tiles ? tiles : 1);
        float *qf = (float *)malloc(hd * sizeof(float));
        float *acc = (float *)malloc(hd * sizeof(float));
#pragma omp for schedule(dynamic, 4)
        for (size_t i = 0; i < rows * heads; i++) {
            const size_t row = i / heads, head = i % heads;
            const size_t block = row / 128;
            memset(keep, 0, tiles ? tiles : 1);
            size_t count = ptr[block + 1] - ptr[block];
            if (count > tiles) count = tiles;
            for (size_t t = 0; t < count; t++) keep[idx[ptr[block] + t]] = 1;
            const size_t qb = (row * heads + head) * hd;
            for (size_t d = 0; d < hd; d++) qf[d] = b2f(q[qb + d]);
            float mx = -INFINITY;
            for (size_t j = 0; j < rows; j++) {
                if (!keep[j / 64]) continue;
                const bf16 *kr = k + (j * heads + head) * hd;
                float dot = 0.0f;
                for (size_t d = 0; d < hd; d++) dot = fmaf(qf[d], b2f(kr[d]), dot);
                s[j] = dot * scale;
                if (s[j] > mx) mx = s[j];
            }
            float l = 0.0f;
            for (size_t j = 0; j < rows; j++) {
                if (!keep[j / 64]) continue;
                s[j] = expf(s[j] - mx);
                l += s[j];
            }
            const float inv = l > 0.0f ? 1.0f / l : 0.0f;
            for (size_t d = 0; d < hd; d++) acc[d] = 0.0f;
            for (size_t j = 0; j < rows; j++) {
                if (!keep[j / 64]) continue;
                const bf16 *vr = v + (j * heads + head) * hd;
                const float p = round_p ? rbf(s[j]) : s[j] * inv;
                for (size_t d = 0; d < hd; d++)
                    acc[d] = fmaf(p, b2f(vr[d]), acc[d]);
            }
            const size_t ob = head_major ? (head * rows + row) * hd : qb;
            for (size_t d = 0; d < hd; d++)
                out[ob + d] = f2b(round_p ? acc[d] * inv : acc[d]);
        }
        free(s);
        free(keep);
        free(qf);
        free(acc);
    }
}

/* Token reduction (reference h3_cuda_dit.cu:336-360, 410-439): pool rows
 * pair.x / pair.y of the grid into one reduced row (their f32 mean rounded
 * to bf16, or the single row when they coincide), snapshotting the source
 * rows into original and the pooled row into baseline[baseline_index]. */
void orc_token_pool(const bf16 *input, const uint32_t *pairs, bf16 *output,
                    bf16 *baseline, const uint32_t *baseline_indices,
                    bf16 *original, size_t rows, size_t width) {
    for (size_t r = 0; r < rows; r++) {
        const uint32_t x = pairs[2 * r], y = pairs[2 * r + 1];
        for (size_t c = 0; c < width; c++) {
            const bf16 first = input[(size_t)x * width + c];
            original[(size_t)x * width + c] = first;
            bf16 pooled = first;
            if (x != y) {
                const bf16 second = input[(size_t)y * width + c];
                original[(size_t)y * width + c] = second;
                pooled = f2b((b2f(first) + b2f(second)) * 0.5f);
            }
            output[r * width + c] = pooled;
            if (baseline_indices[r] != 0xffffffffu)
                baseline[(size_t)baseline_indices[r] * width + c] = pooled;
        }
    }
}

/* Token expansion (reference h3_cuda_dit.cu:441-470): full row r takes its
 * parent's reduced row directly (exact prefix, or no baseline), else
 * bf16(original + scale * (reduced - baseline)) with the FMA the kernel's
 * a * b + c contracts to. */
void orc_token_expand(const bf16 *original, const bf16 *reduced,
                      const bf16 *baseline, const uint32_t *baseline_indices,
                      const uint32_t *parents, bf16 *output, size_t rows,
                      size_t width, size_t exact_prefix_rows,
                      float update_scale) {
    for (size_t r = 0; r < rows; r++) {
        const uint32_t parent = parents[r];
        const uint32_t b = baseline_indices[parent];
        for (size_t c = 0; c < width; c++) {
            const bf16 red = reduced[(size_t)parent * width + c];
            if (r < exact_prefix_rows || b == 0xffffffffu) {
                output[r * width + c] = red;
                continue;
            }
            const float update = b2f(red) - b2f(baseline[(size_t)b * width + c]);
            output[r * width + c] =
                f2b(fmaf(update_scale, update, b2f(original[r * width + c])));
        }
    }
}

/* ------------------------------------------------------- elementwise */

static inline float silu(float x) { return x / (1.0f + expf(-x)); }

/* GELU tanh form with the reference's saturation (h3_cuda_core.cu:139-158) */
static inline float gelu_tanh(float x) {
    float inner = 0.7978845608028654f * (x + 0.044715f * x * x * x);
    return inner <= -10.0f ? 0.0f
         : inner >= 10.0f  ? x
                           : 0.5f * x * (1.0f + tanhf(inner));
}

/* SwiGLU over fused [rows][2 width] (h3_cuda_core.cu:104-114) */
void orc_swiglu(const bf16 *fused, bf16 *out, size_t rows, size_t width) {
#pragma omp parallel for schedule(static)
    for (size_t r = 0; r < rows; r++)
        for (size_t c = 0; c < width; c++) {
            float g = b2f(fused[r * 2 * width + c]);
            float u = b2f(fused[r * 2 * width + width + c]);
            out[r * width + c] = f2b(silu(g) * u);
        }
}

void orc_gelu(const bf16 *in, bf16 *out, size_t n) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; i++) out[i] = f2b(gelu_tanh(b2f(in[i])));
}

void orc_silu(const bf16 *in, bf16 *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = f2b(silu(b2f(in[i])));
}

void orc_add(const bf16 *a, const bf16 *b, bf16 *out, size_t n) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; i++) out[i] = f2b(b2f(a[i]) + b2f(b[i]));
}

void orc_sub(const bf16 *a, const bf16 *b, bf16 *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = f2b(b2f(a[i]) - b2f(b[i]));
}

/* Euler step (h3_cuda_dit.cu:536-548) */
void orc_euler(float *sample, const bf16 *last, const bf16 *prev, size_t n,
               float delta, float ratio) {
    for (size_t i = 0; i < n; i++) {
        float v = b2f(last[i]);
        float vel = fmaf(ratio, v - b2f(prev[i]), v);
        sample[i] = fmaf(delta, vel, sample[i]);
    }
}

/* Final adaLN head (h3_cuda_dit.cu:179-234): inverse RMS, bf16-rounded adaLN
 * row, then bias + sequential fmaf dot with each output column. */
void orc_adaln_linear(const bf16 *x, const bf16 *nw, const bf16 *mod,
                      const uint32_t *map, const bf16 *w, const bf16 *bias,
                      bf16 *out, float *inverse, size_t rows, size_t width,
                      size_t n, size_t slots, size_t shift_slot,
                      size_t scale_slot, float eps) {
#pragma omp parallel
    {
        float *v = (float *)malloc(width * sizeof(float));
#pragma omp for schedule(static)
        for (size_t r = 0; r < rows; r++) {
            for (size_t c = 0; c < width; c++) v[c] = b2f(x[r * width + c]);
            const float inv = row_inverse_rms(v, width, eps);
            if (inverse) inverse[r] = inv;
            const bf16 *m = mod + (size_t)map[r] * slots * width;
            for (size_t c = 0; c < width; c++) {
                float nrm = v[c] * inv * b2f(nw[c]);
                v[c] = rbf(nrm * (1.0f + b2f(m[scale_slot * width + c])) +
                           b2f(m[shift_slot * width + c]));
            }
            for (size_t j = 0; j < n; j++) {
                float sum = bias ? b2f(bias[j]) : 0.0f;
                for (size_t c = 0; c < width; c++)
                    sum = fmaf(v[c], b2f(w[j * width + c]), sum);
                out[r * n + j] = f2b(sum);
            }
        }
        free(v);
    }
}
