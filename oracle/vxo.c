/*
 * vxo — CPU oracle for the speculative-decoding verify path (TEST
 * INFRASTRUCTURE ONLY; see vxo.h for who may load it).
 *
 * Restates, in plain C and in the reference's loop order:
 *   src/paged/metal_kernels.rs  qmm_4bit_cpu :2325-2367,
 *                               paged_decode_attention_cpu :2374-2438,
 *                               MSL paged_prefill_attention :307-395 (visibility),
 *                               MSL batched_rope_decode :209-241,
 *                               MSL batched_scatter :251-279
 *   src/paged/qwen3.rs          RotaryEmbedding::new :278-295, Qwen3MLP :333-339,
 *                               PagedQwen3Attention::forward :418-480 + :657-760,
 *                               DecoderLayer::forward :932-939,
 *                               PagedQwen3::forward / forward_all :994-1036
 *   src/paged/spec.rs           SpecEngine::prefill :131-182, step :186-316,
 *                               ensure_capacity :337-349, argmax_slice :356-366
 *   src/paged/pages.rs          PagedKvCache alloc/free :93-234
 *   src/paged/dyn_quant.rs      pack_int4_into_u32 :125-151
 * Compile with -ffp-contract=off (see Makefile).
 */
#include "vxo.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static __thread char g_err[512];
static int set_err(const char *msg) {
    snprintf(g_err, sizeof g_err, "%s", msg);
    return -1;
}
const char *vxo_last_error(void) { return g_err; }

/* ------------------------------------------------------------------------ */
/* storage rounding                                                          */
/* ------------------------------------------------------------------------ */
static uint32_t f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static float u2f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t vxo_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 -> inf */
    if (ax < 0x33000000u) return (uint16_t)sign;              /* < 2^-25 -> 0 */
    int e = (int)(ax >> 23) - 127;
    uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    if (e >= -14) {
        uint32_t h = ((uint32_t)(e + 15) << 10) | ((mant >> 13) & 0x3ffu);
        uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    /* subnormal result: units of 2^-24 */
    int s = -e - 1; /* 14..24 */
    uint32_t h = mant >> s;
    uint32_t rem = mant & ((1u << s) - 1u);
    uint32_t half = 1u << (s - 1);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float vxo_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0) {
        if (m == 0) return u2f(sign);
        float v = (float)m * (1.0f / 16777216.0f); /* exact */
        return sign ? -v : v;
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t vxo_f32_to_bf16(float f) {
    uint32_t x = f2u(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    uint32_t r = x + 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(r >> 16);
}

float vxo_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

float vxo_round(float x, int dtype) {
    if (dtype == VXO_F16) return vxo_f16_to_f32(vxo_f32_to_f16(x));
    if (dtype == VXO_BF16) return vxo_bf16_to_f32(vxo_f32_to_bf16(x));
    return x;
}

void vxo_round_array(float *x, int64_t n, int dtype) {
    if (dtype == VXO_F32) return;
    for (int64_t i = 0; i < n; i++) x[i] = vxo_round(x[i], dtype);
}

/* ------------------------------------------------------------------------ */
/* Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11)                         */
/* ------------------------------------------------------------------------ */
void vxo_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int r = 0; r < 10; r++) {
        uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
        uint32_t n1 = (uint32_t)p1;
        uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        uint32_t n3 = (uint32_t)p0;
        c0 = n0;
        c1 = n1;
        c2 = n2;
        c3 = n3;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    out[0] = c0;
    out[1] = c1;
    out[2] = c2;
    out[3] = c3;
}

float vxo_u01(uint32_t x) { return (float)(x >> 8) * (1.0f / 16777216.0f); }

void vxo_spec_uniforms(uint64_t seed, uint32_t stream0, uint32_t round, int64_t batch,
                       int64_t k, float *out) {
    uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    for (int64_t b = 0; b < batch; b++)
        for (int64_t i = 0; i <= k; i++) {
            uint32_t ctr[4] = {stream0 + (uint32_t)b, round, (uint32_t)i, 0u};
            uint32_t r[4];
            vxo_philox4x32_10(ctr, key, r);
            float *o = out + (b * (k + 1) + i) * 4;
            for (int j = 0; j < 4; j++) o[j] = vxo_u01(r[j]);
        }
}

/* ------------------------------------------------------------------------ */
/* Deterministic exp: Cody-Waite reduction x = k ln2 + r, degree-7 Taylor    */
/* polynomial in Horner form for e^r on |r| <= ln2/2, scale by 2^k.  Every   */
/* step is one IEEE single operation so host and device agree bit-for-bit.   */
/* ------------------------------------------------------------------------ */
float vxo_expf(float x) {
    if (x != x) return x;
    if (x > 88.5f) return INFINITY;
    if (x < -87.0f) return 0.0f;
    const float log2e = 1.44269502925872802734375f; /* 0x3FB8AA3B */
    const float ln2_hi = 0.693145751953125f;        /* 0x3F317200 */
    const float ln2_lo = 1.428606765330187e-06f;    /* ln2 - ln2_hi */
    float kf = rintf(x * log2e);
    float r = x - kf * ln2_hi;
    r = r - kf * ln2_lo;
    float p = 1.98412701138295233249664306640625e-04f; /* 1/5040 */
    p = p * r + 1.38888892345130443572998046875e-03f;  /* 1/720 */
    p = p * r + 8.33333376795053482055664062500e-03f;  /* 1/120 */
    p = p * r + 4.16666679084300994873046875000e-02f;  /* 1/24 */
    p = p * r + 1.66666671633720397949218750000e-01f;  /* 1/6 */
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    int k = (int)kf;
    if (k > 127) {
        p = p * u2f((uint32_t)(127 + 127) << 23);
        k -= 127;
    }
    return p * u2f((uint32_t)(k + 127) << 23);
}

/* ------------------------------------------------------------------------ */
/* int4 packing                                                              */
/* ------------------------------------------------------------------------ */
void vxo_pack_int4(const uint32_t *codes, int64_t n, int64_t k, uint32_t *packed) {
    for (int64_t r = 0; r < n; r++)
        for (int64_t c = 0; c < k; c += 8) {
            const uint32_t *h = codes + r * k + c;
            uint32_t p = 0;
            for (int b = 0; b < 8; b++) p |= (h[b] & 0xFu) << (4 * b);
            packed[r * (k / 8) + c / 8] = p;
        }
}

void vxo_unpack_int4(const uint32_t *packed, int64_t n, int64_t k, uint32_t *codes) {
    for (int64_t r = 0; r < n; r++)
        for (int64_t c = 0; c < k; c++)
            codes[r * k + c] = (packed[r * (k / 8) + c / 8] >> (4 * (c % 8))) & 0xFu;
}

/* ------------------------------------------------------------------------ */
/* qmm_4bit_cpu                                                              */
/* ------------------------------------------------------------------------ */
int vxo_qmm_4bit(const float *x, const uint32_t *qweight, const float *scales,
                 const float *biases, const float *bias_vec, float *out, int64_t m, int64_t n,
                 int64_t k, int64_t gs, int threads) {
    if (k % 8 != 0) return set_err("qmm_4bit: K must be a multiple of 8");
    if (gs == 0 || gs % 8 != 0 || k % gs != 0)
        return set_err("qmm_4bit: group_size must be a multiple of 8 and divide K");
    const int64_t k_packed = k / 8, k_groups = k / gs;
    if (threads < 1) threads = 1;
    /* Each output keeps the reference's accumulation: zero, then x*w over k
     * in (group, word, nibble) order, then the bias.  The rows of one output
     * column are independent sums, so they run side by side over a
     * transposed X (xT[k][m]), which vectorises across rows without
     * reassociating any sum. */
    float *xT = (float *)malloc(sizeof(float) * (size_t)(m * k));
    if (!xT) return set_err("qmm_4bit: oom");
    for (int64_t mi = 0; mi < m; mi++)
        for (int64_t kk = 0; kk < k; kk++) xT[kk * m + mi] = x[mi * k + kk];
    int oom = 0;
#pragma omp parallel num_threads(threads)
    {
        float *acc = (float *)malloc(sizeof(float) * (size_t)m);
        if (!acc) {
#pragma omp atomic write
            oom = 1;
        }
#pragma omp for schedule(static)
        for (int64_t ni = 0; ni < n; ni++) {
            if (!acc) continue;
            for (int64_t mi = 0; mi < m; mi++) acc[mi] = 0.0f;
            for (int64_t kg = 0; kg < k_groups; kg++) {
                const float scale = scales[ni * k_groups + kg];
                const float bias = biases[ni * k_groups + kg];
                for (int64_t kp = 0; kp < gs / 8; kp++) {
                    const uint32_t pkg = qweight[ni * k_packed + kg * (gs / 8) + kp];
                    for (int b = 0; b < 8; b++) {
                        const float q = (float)((pkg >> (b * 4)) & 0xFu);
                        const float w = q * scale + bias;
                        const float *xc = xT + (kg * gs + kp * 8 + b) * m;
                        for (int64_t mi = 0; mi < m; mi++) acc[mi] += xc[mi] * w;
                    }
                }
            }
            if (bias_vec)
                for (int64_t mi = 0; mi < m; mi++) acc[mi] += bias_vec[ni];
            for (int64_t mi = 0; mi < m; mi++) out[mi * n + ni] = acc[mi];
        }
        free(acc);
    }
    free(xT);
    if (oom) return set_err("qmm_4bit: oom");
    return 0;
}

/* ------------------------------------------------------------------------ */
/* paged attention                                                           */
/* ------------------------------------------------------------------------ */
int vxo_paged_attention(const float *q, const float *k_pool, const float *v_pool,
                        const uint32_t *block_table, int64_t max_blocks,
                        const uint32_t *cu_seqlens, const uint32_t *kv_offsets,
                        int64_t n_seqs, const uint64_t *tree_mask, int64_t total_q,
                        int64_t h_q, int64_t h_kv, int64_t d, int64_t ps, float scale,
                        uint32_t sliding_window, float *out) {
    if (h_kv <= 0 || h_q % h_kv != 0) return set_err("attention: H_q must be divisible by H_kv");
    const int64_t groups = h_q / h_kv;
    /* block-table bounds first (same visiting rule as the main loop), so the
     * rows can then run in parallel: each output element keeps the serial
     * per-row online-softmax order of paged_decode_attention_cpu */
    for (int64_t row = 0; row < total_q; row++) {
        int64_t seq = 0;
        while (seq + 1 < n_seqs && (int64_t)cu_seqlens[seq + 1] <= row) seq++;
        const int64_t t = row - cu_seqlens[seq];
        const int64_t off = kv_offsets[seq];
        const int64_t r_seq = (int64_t)cu_seqlens[seq + 1] - (int64_t)cu_seqlens[seq];
        const int64_t end = tree_mask ? off + r_seq : off + t + 1;
        const int64_t self_len = off + t + 1;
        const int64_t w = sliding_window;
        const int64_t start = (w > 0 && self_len > w) ? self_len - w : 0;
        for (int64_t pos = start; pos < end; pos++) {
            if (tree_mask && pos >= off) {
                const int64_t j = pos - off;
                if (j >= 64 || !((tree_mask[row] >> j) & 1ull)) continue;
            }
            if (pos / ps >= max_blocks) return set_err("attention: block_table too short");
        }
    }
    int oom = 0;
#pragma omp parallel
    {
        float *acc = (float *)malloc(sizeof(float) * (size_t)d);
        if (!acc) {
#pragma omp atomic write
            oom = 1;
        }
#pragma omp for schedule(dynamic, 1)
        for (int64_t row = 0; row < total_q; row++) {
            if (!acc) continue;
            int64_t seq = 0;
            while (seq + 1 < n_seqs && (int64_t)cu_seqlens[seq + 1] <= row) seq++;
            const int64_t t = row - cu_seqlens[seq];
            const int64_t off = kv_offsets[seq];
            const int64_t r_seq = (int64_t)cu_seqlens[seq + 1] - (int64_t)cu_seqlens[seq];
            /* last visible position + 1 */
            const int64_t end = tree_mask ? off + r_seq : off + t + 1;
            const int64_t self_len = off + t + 1;
            const int64_t w = sliding_window;
            const int64_t start = (w > 0 && self_len > w) ? self_len - w : 0;
            for (int64_t hq = 0; hq < h_q; hq++) {
                const int64_t hk = hq / groups;
                float m = -INFINITY, l = 0.0f;
                for (int64_t i = 0; i < d; i++) acc[i] = 0.0f;
                const float *qr = q + (row * h_q + hq) * d;
                for (int64_t pos = start; pos < end; pos++) {
                    if (tree_mask && pos >= off) {
                        const int64_t j = pos - off;
                        if (j >= 64 || !((tree_mask[row] >> j) & 1ull)) continue;
                    }
                    const int64_t blk = pos / ps;
                    const int64_t page = block_table[seq * max_blocks + blk];
                    const int64_t base = page * (h_kv * ps * d) + hk * (ps * d) + (pos % ps) * d;
                    float s = 0.0f;
                    for (int64_t i = 0; i < d; i++) s += qr[i] * k_pool[base + i];
                    s *= scale;
                    const float new_m = fmaxf(m, s);
                    const float alpha = expf(m - new_m);
                    const float beta = expf(s - new_m);
                    for (int64_t i = 0; i < d; i++) acc[i] = acc[i] * alpha + beta * v_pool[base + i];
                    l = l * alpha + beta;
                    m = new_m;
                }
                float *o = out + (row * h_q + hq) * d;
                for (int64_t i = 0; i < d; i++) o[i] = acc[i] / l;
            }
        }
        free(acc);
    }
    if (oom) return set_err("attention: oom");
    return 0;
}

/* ------------------------------------------------------------------------ */
/* RoPE, scatter, norms                                                      */
/* ------------------------------------------------------------------------ */
void vxo_rope_tables(int64_t max_pos, int64_t dim, double theta, float *cos_t, float *sin_t) {
    const int64_t half = dim / 2;
    float *inv = (float *)malloc(sizeof(float) * (size_t)half);
    for (int64_t j = 0; j < half; j++)
        inv[j] = 1.0f / (float)pow(theta, (double)(2 * j) / (double)dim);
    for (int64_t t = 0; t < max_pos; t++)
        for (int64_t j = 0; j < half; j++) {
            const float f = (float)t * inv[j];
            cos_t[t * half + j] = cosf(f);
            sin_t[t * half + j] = sinf(f);
        }
    free(inv);
}

void vxo_rope_apply(float *x, const float *cos_t, const float *sin_t, const uint32_t *pos,
                    int64_t n, int64_t h, int64_t d, int dtype) {
    const int64_t half = d / 2;
    for (int64_t r = 0; r < n; r++)
        for (int64_t hh = 0; hh < h; hh++) {
            float *b = x + (r * h + hh) * d;
            for (int64_t j = 0; j < half; j++) {
                const float x1 = b[j], x2 = b[j + half];
                const float c = cos_t[(int64_t)pos[r] * half + j];
                const float s = sin_t[(int64_t)pos[r] * half + j];
                b[j] = vxo_round(x1 * c - x2 * s, dtype);
                b[j + half] = vxo_round(x1 * s + x2 * c, dtype);
            }
        }
}

void vxo_kv_scatter(float *pool, const float *values, const uint32_t *page_ids,
                    const uint32_t *slots, int64_t n, int64_t h, int64_t s, int64_t d) {
    for (int64_t r = 0; r < n; r++)
        for (int64_t hh = 0; hh < h; hh++)
            memcpy(pool + (int64_t)page_ids[r] * (h * s * d) + hh * (s * d) + (int64_t)slots[r] * d,
                   values + (r * h + hh) * d, sizeof(float) * (size_t)d);
}

void vxo_rmsnorm(const float *x, const float *w, float *y, int64_t rows, int64_t dim, float eps,
                 int dtype) {
    for (int64_t r = 0; r < rows; r++) {
        const float *xr = x + r * dim;
        float sum2 = 0.0f;
        for (int64_t i = 0; i < dim; i++) sum2 += xr[i] * xr[i];
        const float m = sqrtf(sum2 / (float)dim + eps);
        for (int64_t i = 0; i < dim; i++) y[r * dim + i] = vxo_round(xr[i] / m * w[i], dtype);
    }
}

float vxo_silu(float x) { return x / (1.0f + expf(-x)); }

/* ------------------------------------------------------------------------ */
/* acceptance                                                                */
/* ------------------------------------------------------------------------ */
uint32_t vxo_argmax(const float *v, int64_t n) {
    uint32_t best_i = 0;
    float best_v = -INFINITY;
    for (int64_t i = 0; i < n; i++)
        if (v[i] > best_v) {
            best_v = v[i];
            best_i = (uint32_t)i;
        }
    return best_i;
}

void vxo_accept_greedy(const float *logits, int64_t vocab, const uint32_t *cand, int64_t batch,
                       int64_t k, int32_t *accepted, uint32_t *tokens) {
    for (int64_t b = 0; b < batch; b++) {
        const float *lb = logits + b * (k + 1) * vocab;
        int64_t a = 0;
        while (a < k && cand[b * k + a] == vxo_argmax(lb + a * vocab, vocab)) a++;
        for (int64_t i = 0; i < a; i++) tokens[b * (k + 1) + i] = cand[b * k + i];
        tokens[b * (k + 1) + a] = vxo_argmax(lb + a * vocab, vocab);
        accepted[b] = (int32_t)a;
    }
}

static float tree_sum_256(float *s) {
    for (int stride = VXO_SM_THREADS / 2; stride >= 1; stride >>= 1)
        for (int t = 0; t < stride; t++) s[t] = s[t] + s[t + stride];
    return s[0];
}

void vxo_row_softmax_stats(const float *row, int64_t vocab, float inv_t, float *m_out,
                           float *z_out) {
    const int64_t nch = (vocab + VXO_SM_CHUNK - 1) / VXO_SM_CHUNK;
    float *mc = (float *)malloc(sizeof(float) * (size_t)nch);
    float *zc = (float *)malloc(sizeof(float) * (size_t)nch);
    float part[VXO_SM_THREADS];
    for (int64_t c = 0; c < nch; c++) {
        const int64_t lo = c * VXO_SM_CHUNK;
        const int64_t hi = lo + VXO_SM_CHUNK < vocab ? lo + VXO_SM_CHUNK : vocab;
        float m = -INFINITY;
        for (int64_t j = lo; j < hi; j++) m = fmaxf(m, row[j]);
        /* a chunk with no finite maximum holds no probability mass (its
         * (row[j] - m) would be -inf - -inf) */
        for (int t = 0; t < VXO_SM_THREADS; t++) {
            float s = 0.0f;
            if (m != -INFINITY)
                for (int64_t j = lo + t; j < hi; j += VXO_SM_THREADS) s = s + vxo_expf((row[j] - m) * inv_t);
            part[t] = s;
        }
        mc[c] = m;
        zc[c] = tree_sum_256(part);
    }
    float M = -INFINITY;
    for (int64_t c = 0; c < nch; c++) M = fmaxf(M, mc[c]);
    float Z = 0.0f;
    for (int64_t c = 0; c < nch; c++)
        if (mc[c] != -INFINITY) Z = Z + zc[c] * vxo_expf((mc[c] - M) * inv_t);
    *m_out = M;
    *z_out = Z;
    free(mc);
    free(zc);
}

static float resid_elem(const float *lt, float mt, float zt, const float *ld, float md, float zd,
                        float inv_t, int64_t j) {
    /* a row with no finite logit has no mass anywhere */
    const float p = mt == -INFINITY ? 0.0f : vxo_expf((lt[j] - mt) * inv_t) / zt;
    if (!ld) return p;
    const float q = md == -INFINITY ? 0.0f : vxo_expf((ld[j] - md) * inv_t) / zd;
    const float d = p - q;
    return d > 0.0f ? d : 0.0f;
}

uint32_t vxo_sample_residual(const float *lt, float mt, float zt, const float *ld, float md,
                             float zd, int64_t vocab, float inv_t, float u) {
    const int64_t nch = (vocab + VXO_SM_CHUNK - 1) / VXO_SM_CHUNK;
    const int64_t nsub_per = VXO_SM_CHUNK / VXO_SM_SUB;
    /* sub-chunk sums, chunk sums, total: each sequential in index order */
    const int64_t nsub = nch * nsub_per;
    float *ss = (float *)calloc((size_t)nsub, sizeof(float));
    float *cs = (float *)calloc((size_t)nch, sizeof(float));
    int64_t last_pos = -1;
    for (int64_t sidx = 0; sidx < nsub; sidx++) {
        const int64_t lo = sidx * VXO_SM_SUB;
        float s = 0.0f;
        for (int64_t j = lo; j < lo + VXO_SM_SUB && j < vocab; j++) {
            const float r = resid_elem(lt, mt, zt, ld, md, zd, inv_t, j);
            if (r > 0.0f) last_pos = j;
            s = s + r;
        }
        ss[sidx] = s;
    }
    for (int64_t c = 0; c < nch; c++) {
        float s = 0.0f;
        for (int64_t i = 0; i < nsub_per; i++) s = s + ss[c * nsub_per + i];
        cs[c] = s;
    }
    float total = 0.0f;
    for (int64_t c = 0; c < nch; c++) total = total + cs[c];
    const float target = u * total;
    uint32_t result = (uint32_t)(last_pos < 0 ? 0 : last_pos);
    float run = 0.0f;
    for (int64_t c = 0; c < nch; c++) {
        if (run + cs[c] > target) {
            /* inside chunk c */
            int64_t found = -1, last_in_chunk = -1;
            float run2 = run;
            for (int64_t i = 0; i < nsub_per && found < 0; i++) {
                const int64_t sidx = c * nsub_per + i;
                if (run2 + ss[sidx] > target) {
                    float run3 = run2;
                    const int64_t lo = sidx * VXO_SM_SUB;
                    for (int64_t j = lo; j < lo + VXO_SM_SUB && j < vocab; j++) {
                        const float r = resid_elem(lt, mt, zt, ld, md, zd, inv_t, j);
                        if (r > 0.0f) last_in_chunk = j;
                        run3 = run3 + r;
                        if (run3 > target) {
                            found = j;
                            break;
                        }
                    }
                    if (found < 0) {
                        /* rounding: fall back to last positive element of the chunk */
                        for (int64_t j = (c + 1) * VXO_SM_CHUNK - 1; j >= c * VXO_SM_CHUNK; j--)
                            if (j < vocab && resid_elem(lt, mt, zt, ld, md, zd, inv_t, j) > 0.0f) {
                                found = j;
                                break;
                            }
                    }
                    break;
                }
                run2 = run2 + ss[sidx];
            }
            if (found < 0) {
                for (int64_t j = (c + 1) * VXO_SM_CHUNK - 1; j >= c * VXO_SM_CHUNK; j--)
                    if (j < vocab && resid_elem(lt, mt, zt, ld, md, zd, inv_t, j) > 0.0f) {
                        found = j;
                        break;
                    }
            }
            (void)last_in_chunk;
            if (found >= 0) result = (uint32_t)found;
            break;
        }
        run = run + cs[c];
    }
    free(ss);
    free(cs);
    return result;
}

static float prob_of(const float *row, float m, float z, float inv_t, uint32_t tok) {
    return m == -INFINITY ? 0.0f : vxo_expf((row[tok] - m) * inv_t) / z;
}

void vxo_sample_draft(const float *draft_logits, const float *uniforms, int64_t batch, int64_t k,
                      int64_t vocab, float inv_t, uint32_t *candidates) {
    for (int64_t b = 0; b < batch; b++)
        for (int64_t i = 0; i < k; i++) {
            const float *row = draft_logits + (b * k + i) * vocab;
            float m, z;
            vxo_row_softmax_stats(row, vocab, inv_t, &m, &z);
            candidates[b * k + i] = vxo_sample_residual(row, m, z, NULL, 0.0f, 1.0f, vocab, inv_t,
                                                        uniforms[(b * (k + 1) + i) * 4 + 0]);
        }
}

void vxo_accept_stochastic(const float *tl, const float *dl, const uint32_t *cand,
                           const float *uni, int64_t batch, int64_t k, int64_t vocab, float inv_t,
                           int32_t *accepted, uint32_t *tokens) {
    for (int64_t b = 0; b < batch; b++) {
        int64_t a = 0;
        uint32_t next = 0;
        for (; a < k; a++) {
            const float *tr = tl + (b * (k + 1) + a) * vocab;
            const float *dr = dl + (b * k + a) * vocab;
            float mt, zt, md, zd;
            vxo_row_softmax_stats(tr, vocab, inv_t, &mt, &zt);
            vxo_row_softmax_stats(dr, vocab, inv_t, &md, &zd);
            const uint32_t c = cand[b * k + a];
            const float p = prob_of(tr, mt, zt, inv_t, c);
            const float q = prob_of(dr, md, zd, inv_t, c);
            const float ratio = p / q;
            const float acc = ratio < 1.0f ? ratio : 1.0f;
            const float u = uni[(b * (k + 1) + a) * 4 + 1];
            if (!(u < acc)) {
                next = vxo_sample_residual(tr, mt, zt, dr, md, zd, vocab, inv_t,
                                           uni[(b * (k + 1) + a) * 4 + 2]);
                break;
            }
            tokens[b * (k + 1) + a] = c;
        }
        if (a == k) {
            const float *tr = tl + (b * (k + 1) + k) * vocab;
            float mt, zt;
            vxo_row_softmax_stats(tr, vocab, inv_t, &mt, &zt);
            next = vxo_sample_residual(tr, mt, zt, NULL, 0.0f, 1.0f, vocab, inv_t,
                                       uni[(b * (k + 1) + k) * 4 + 2]);
        }
        tokens[b * (k + 1) + a] = next;
        accepted[b] = (int32_t)a;
    }
}

void vxo_tree_masks(const int32_t *parents, int64_t r, uint64_t *masks, int32_t *depth) {
    for (int64_t i = 0; i < r; i++) {
        uint64_t m = 1ull << i;
        int32_t dd = 0;
        for (int32_t p = parents[i]; p >= 0; p = parents[p]) {
            m |= 1ull << p;
            dd++;
        }
        if (masks) masks[i] = m;
        if (depth) depth[i] = dd;
    }
}

void vxo_accept_tree(const float *logits, const int32_t *parents, const uint32_t *node_tokens,
                     int64_t batch, int64_t r, int64_t vocab, int32_t *accepted, int32_t *path,
                     uint32_t *tokens) {
    for (int64_t b = 0; b < batch; b++) {
        const float *lb = logits + b * r * vocab;
        int32_t cur = 0;
        int64_t a = 0;
        path[b * r + 0] = 0;
        for (;;) {
            const uint32_t t = vxo_argmax(lb + cur * vocab, vocab);
            int32_t next = -1;
            for (int64_t j = cur + 1; j < r; j++)
                if (parents[j] == cur && node_tokens[b * r + j] == t) {
                    next = (int32_t)j;
                    break;
                }
            if (next < 0) break;
            tokens[b * r + a] = t;
            a++;
            path[b * r + a] = next;
            cur = next;
        }
        tokens[b * r + a] = vxo_argmax(lb + cur * vocab, vocab);
        accepted[b] = (int32_t)a;
    }
}

/* ------------------------------------------------------------------------ */
/* pages                                                                     */
/* ------------------------------------------------------------------------ */
struct vxo_pages {
    int64_t layers, kv_heads, head_dim, page_size, num_pages;
    float **pools; /* [layers * 2] */
    uint32_t *free_list;
    int64_t n_free;
    uint32_t *refcount;
};

vxo_pages *vxo_pages_create(int64_t layers, int64_t kv_heads, int64_t head_dim, int64_t page_size,
                            int64_t num_pages) {
    if (layers <= 0 || num_pages <= 0) {
        set_err("PagedKvCache must have >=1 layer and >=1 page");
        return NULL;
    }
    vxo_pages *p = (vxo_pages *)calloc(1, sizeof *p);
    p->layers = layers;
    p->kv_heads = kv_heads;
    p->head_dim = head_dim;
    p->page_size = page_size;
    p->num_pages = num_pages;
    p->pools = (float **)calloc((size_t)(layers * 2), sizeof(float *));
    const size_t per = (size_t)(num_pages * kv_heads * page_size * head_dim);
    for (int64_t i = 0; i < layers * 2; i++) {
        p->pools[i] = (float *)calloc(per, sizeof(float));
        if (!p->pools[i]) {
            set_err("pages: oom");
            vxo_pages_destroy(p);
            return NULL;
        }
    }
    p->free_list = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)num_pages);
    for (int64_t i = 0; i < num_pages; i++) p->free_list[i] = (uint32_t)(num_pages - 1 - i);
    p->n_free = num_pages;
    p->refcount = (uint32_t *)calloc((size_t)num_pages, sizeof(uint32_t));
    return p;
}

void vxo_pages_destroy(vxo_pages *p) {
    if (!p) return;
    if (p->pools)
        for (int64_t i = 0; i < p->layers * 2; i++) free(p->pools[i]);
    free(p->pools);
    free(p->free_list);
    free(p->refcount);
    free(p);
}

int vxo_pages_alloc(vxo_pages *p, int64_t n, uint32_t *out) {
    if (p->n_free < n) return set_err("alloc: not enough free pages");
    for (int64_t i = 0; i < n; i++) {
        const uint32_t pg = p->free_list[--p->n_free];
        p->refcount[pg] = 1;
        out[i] = pg;
    }
    return 0;
}

void vxo_pages_free(vxo_pages *p, const uint32_t *pages, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        const uint32_t pg = pages[i];
        if ((int64_t)pg >= p->num_pages) continue;
        const uint32_t prev = p->refcount[pg];
        if (prev == 0) continue;
        p->refcount[pg] = prev - 1;
        if (prev == 1) p->free_list[p->n_free++] = pg;
    }
}

int64_t vxo_pages_num_free(const vxo_pages *p) { return p->n_free; }

float *vxo_pages_pool(vxo_pages *p, int64_t layer, int kv) { return p->pools[layer * 2 + kv]; }

/* ------------------------------------------------------------------------ */
/* model                                                                     */
/* ------------------------------------------------------------------------ */
struct vxo_model {
    vxo_config cfg;
    vxo_weights w;
    float *cos_t, *sin_t; /* rounded to T like the reference's tables */
    int threads;
};

vxo_model *vxo_model_create(const vxo_config *cfg, const vxo_weights *w, int threads) {
    vxo_model *m = (vxo_model *)calloc(1, sizeof *m);
    m->cfg = *cfg;
    m->w = *w;
    m->threads = threads < 1 ? 1 : threads;
    const int64_t half = cfg->head_dim / 2;
    m->cos_t = (float *)malloc(sizeof(float) * (size_t)(cfg->max_pos * half));
    m->sin_t = (float *)malloc(sizeof(float) * (size_t)(cfg->max_pos * half));
    vxo_rope_tables(cfg->max_pos, cfg->head_dim, cfg->rope_theta, m->cos_t, m->sin_t);
    vxo_round_array(m->cos_t, cfg->max_pos * half, cfg->dtype);
    vxo_round_array(m->sin_t, cfg->max_pos * half, cfg->dtype);
    return m;
}

void vxo_model_destroy(vxo_model *m) {
    if (!m) return;
    free(m->cos_t);
    free(m->sin_t);
    free(m);
}

static int qlin(const vxo_model *m, const vxo_qlinear *l, const float *x, float *y, int64_t rows,
                int64_t n, int64_t k) {
    int rc = vxo_qmm_4bit(x, l->qweight, l->scales, l->biases, NULL, y, rows, n, k,
                          m->cfg.group_size, m->threads);
    if (rc == 0) vxo_round_array(y, rows * n, m->cfg.dtype);
    return rc;
}

int vxo_forward(vxo_model *mdl, vxo_pages *pages, const uint32_t *ids, const vxo_seq *seqs,
                int64_t n_seqs, int all_rows, const int32_t *tree_parents, float *logits) {
    const vxo_config *c = &mdl->cfg;
    const int T = c->dtype;
    const int64_t H = c->hidden, F = c->inter, D = c->head_dim, HQ = c->n_heads,
                  HK = c->n_kv_heads, V = c->vocab, ps = pages->page_size;
    int64_t total = 0, max_blocks = 1;
    for (int64_t s = 0; s < n_seqs; s++) {
        total += seqs[s].new_tokens;
        if (seqs[s].n_blocks > max_blocks) max_blocks = seqs[s].n_blocks;
        if (tree_parents && seqs[s].new_tokens != seqs[0].new_tokens)
            return set_err("forward: tree verify needs equal node counts");
    }
    const int64_t R = n_seqs ? seqs[0].new_tokens : 0;
    if (tree_parents && R > 64) return set_err("forward: tree larger than 64 nodes");
    uint64_t tmask[64];
    int32_t tdepth[64];
    if (tree_parents) vxo_tree_masks(tree_parents, R, tmask, tdepth);

    uint32_t *rope_pos = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)total);
    uint32_t *page_ids = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)total);
    uint32_t *slots = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)total);
    uint64_t *masks = tree_parents ? (uint64_t *)malloc(sizeof(uint64_t) * (size_t)total) : NULL;
    uint32_t *cu = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)(n_seqs + 1));
    uint32_t *kvo = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)(n_seqs ? n_seqs : 1));
    uint32_t *bt = (uint32_t *)calloc((size_t)(n_seqs * max_blocks + 1), sizeof(uint32_t));
    int rc = 0;
    int64_t row = 0;
    cu[0] = 0;
    for (int64_t s = 0; s < n_seqs; s++) {
        for (int64_t b = 0; b < seqs[s].n_blocks; b++) bt[s * max_blocks + b] = seqs[s].block_table[b];
        for (int64_t t = 0; t < seqs[s].new_tokens; t++, row++) {
            const int64_t slot_pos = seqs[s].kv_offset + t;
            const int64_t blk = slot_pos / ps;
            if (blk >= seqs[s].n_blocks) {
                rc = set_err("fused prefill: block_table too short");
                goto done_meta;
            }
            page_ids[row] = seqs[s].block_table[blk];
            slots[row] = (uint32_t)(slot_pos % ps);
            rope_pos[row] = (uint32_t)(seqs[s].kv_offset + (tree_parents ? tdepth[t] : t));
            if (masks) masks[row] = tmask[t];
        }
        cu[s + 1] = (uint32_t)row;
        kvo[s] = (uint32_t)seqs[s].kv_offset;
    }
done_meta:
    if (rc) {
        free(rope_pos);
        free(page_ids);
        free(slots);
        free(masks);
        free(cu);
        free(kvo);
        free(bt);
        return rc;
    }

    const int64_t QW = HQ * D, KW = HK * D;
    float *h = (float *)malloc(sizeof(float) * (size_t)(total * H));
    float *n1 = (float *)malloc(sizeof(float) * (size_t)(total * (H > QW ? H : QW)));
    float *qb = (float *)malloc(sizeof(float) * (size_t)(total * QW));
    float *kb = (float *)malloc(sizeof(float) * (size_t)(total * KW));
    float *vb = (float *)malloc(sizeof(float) * (size_t)(total * KW));
    float *ab = (float *)malloc(sizeof(float) * (size_t)(total * QW));
    float *ob = (float *)malloc(sizeof(float) * (size_t)(total * H));
    float *gb = (float *)malloc(sizeof(float) * (size_t)(total * F));
    float *ub = (float *)malloc(sizeof(float) * (size_t)(total * F));
    for (int64_t r = 0; r < total; r++) memcpy(h + r * H, mdl->w.embed + (int64_t)ids[r] * H, sizeof(float) * (size_t)H);
    const float scale = 1.0f / sqrtf((float)D);
    const float eps = (float)c->rms_eps;
    for (int64_t L = 0; L < c->layers && rc == 0; L++) {
        const vxo_layer *ly = &mdl->w.layers[L];
        vxo_rmsnorm(h, ly->ln1, n1, total, H, eps, T);
        if ((rc = qlin(mdl, &ly->q, n1, qb, total, QW, H))) break;
        if ((rc = qlin(mdl, &ly->k, n1, kb, total, KW, H))) break;
        if ((rc = qlin(mdl, &ly->v, n1, vb, total, KW, H))) break;
        if (ly->q_norm) vxo_rmsnorm(qb, ly->q_norm, qb, total * HQ, D, eps, T);
        if (ly->k_norm) vxo_rmsnorm(kb, ly->k_norm, kb, total * HK, D, eps, T);
        vxo_rope_apply(qb, mdl->cos_t, mdl->sin_t, rope_pos, total, HQ, D, T);
        vxo_rope_apply(kb, mdl->cos_t, mdl->sin_t, rope_pos, total, HK, D, T);
        vxo_kv_scatter(vxo_pages_pool(pages, L, 0), kb, page_ids, slots, total, HK, ps, D);
        vxo_kv_scatter(vxo_pages_pool(pages, L, 1), vb, page_ids, slots, total, HK, ps, D);
        if ((rc = vxo_paged_attention(qb, vxo_pages_pool(pages, L, 0), vxo_pages_pool(pages, L, 1),
                                      bt, max_blocks, cu, kvo, n_seqs, masks, total, HQ, HK, D,
                                      ps, scale, 0, ab)))
            break;
        vxo_round_array(ab, total * QW, T);
        if ((rc = qlin(mdl, &ly->o, ab, ob, total, H, QW))) break;
        for (int64_t i = 0; i < total * H; i++) h[i] = vxo_round(h[i] + ob[i], T);
        vxo_rmsnorm(h, ly->ln2, n1, total, H, eps, T);
        if ((rc = qlin(mdl, &ly->gate, n1, gb, total, F, H))) break;
        if ((rc = qlin(mdl, &ly->up, n1, ub, total, F, H))) break;
        for (int64_t i = 0; i < total * F; i++)
            gb[i] = vxo_round(vxo_round(vxo_silu(gb[i]), T) * ub[i], T);
        if ((rc = qlin(mdl, &ly->down, gb, ob, total, H, F))) break;
        for (int64_t i = 0; i < total * H; i++) h[i] = vxo_round(h[i] + ob[i], T);
    }
    if (rc == 0) {
        vxo_rmsnorm(h, mdl->w.norm, n1, total, H, eps, T);
        if (all_rows) {
            rc = qlin(mdl, &mdl->w.lm_head, n1, logits, total, V, H);
        } else {
            float *last = (float *)malloc(sizeof(float) * (size_t)(n_seqs * H));
            for (int64_t s = 0; s < n_seqs; s++)
                memcpy(last + s * H, n1 + ((int64_t)cu[s + 1] - 1) * H, sizeof(float) * (size_t)H);
            rc = qlin(mdl, &mdl->w.lm_head, last, logits, n_seqs, V, H);
            free(last);
        }
    }
    free(h);
    free(n1);
    free(qb);
    free(kb);
    free(vb);
    free(ab);
    free(ob);
    free(gb);
    free(ub);
    free(rope_pos);
    free(page_ids);
    free(slots);
    free(masks);
    free(cu);
    free(kvo);
    free(bt);
    return rc;
}

/* ------------------------------------------------------------------------ */
/* spec engine                                                               */
/* ------------------------------------------------------------------------ */
static int grow(vxo_pages *p, uint32_t **blocks, int64_t *nb, int64_t needed) {
    if (*nb >= needed) return 0;
    const int64_t extra = needed - *nb;
    uint32_t *nbuf = (uint32_t *)realloc(*blocks, sizeof(uint32_t) * (size_t)needed);
    if (!nbuf) return set_err("oom");
    *blocks = nbuf;
    if (vxo_pages_alloc(p, extra, nbuf + *nb)) return set_err("alloc extra pages");
    *nb = needed;
    return 0;
}

static void push_tokens(vxo_spec_state *s, const uint32_t *t, int64_t n) {
    s->tokens = (uint32_t *)realloc(s->tokens, sizeof(uint32_t) * (size_t)(s->n_tokens + n));
    memcpy(s->tokens + s->n_tokens, t, sizeof(uint32_t) * (size_t)n);
    s->n_tokens += n;
}

int vxo_spec_prefill(vxo_spec *e, const uint32_t *const *prompts, const int64_t *lens, int64_t n,
                     vxo_spec_state *states) {
    const int64_t ps = e->target_pages->page_size;
    if (e->draft_pages->page_size != ps) return set_err("draft page_size != target page_size");
    if (e->target->cfg.vocab != e->draft->cfg.vocab)
        return set_err("draft vocab_size != target vocab_size");
    int64_t total = 0;
    for (int64_t b = 0; b < n; b++) {
        if (lens[b] < 2) return set_err("speculative prefill requires a prompt with at least 2 tokens");
        total += lens[b] - 1;
    }
    memset(states, 0, sizeof(vxo_spec_state) * (size_t)n);
    for (int64_t b = 0; b < n; b++) {
        const int64_t head = lens[b] - 1;
        const int64_t need = (head + 1 + ps - 1) / ps;
        vxo_spec_state *s = &states[b];
        s->stream_id = (uint32_t)b;
        if (grow(e->target_pages, &s->target_blocks, &s->n_target_blocks, need))
            return set_err("alloc target prefill pages");
        if (grow(e->draft_pages, &s->draft_blocks, &s->n_draft_blocks, need))
            return set_err("alloc draft prefill pages");
        s->kv_len = head;
        s->last_token = prompts[b][head];
        push_tokens(s, prompts[b], lens[b]);
    }
    uint32_t *ids = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)total);
    vxo_seq *ts = (vxo_seq *)malloc(sizeof(vxo_seq) * (size_t)n);
    vxo_seq *ds = (vxo_seq *)malloc(sizeof(vxo_seq) * (size_t)n);
    int64_t o = 0;
    for (int64_t b = 0; b < n; b++) {
        memcpy(ids + o, prompts[b], sizeof(uint32_t) * (size_t)(lens[b] - 1));
        o += lens[b] - 1;
        ts[b] = (vxo_seq){lens[b] - 1, 0, states[b].target_blocks, states[b].n_target_blocks};
        ds[b] = (vxo_seq){lens[b] - 1, 0, states[b].draft_blocks, states[b].n_draft_blocks};
    }
    float *lg = (float *)malloc(sizeof(float) * (size_t)(n * e->target->cfg.vocab));
    int rc = vxo_forward(e->target, e->target_pages, ids, ts, n, 0, NULL, lg);
    if (!rc) rc = vxo_forward(e->draft, e->draft_pages, ids, ds, n, 0, NULL, lg);
    free(lg);
    free(ids);
    free(ts);
    free(ds);
    return rc;
}

int vxo_spec_adopt(vxo_spec *e, const uint32_t *prompt, int64_t len, vxo_spec_state *s) {
    const int64_t ps = e->target_pages->page_size;
    if (len < 2) return set_err("speculative prefill requires a prompt with at least 2 tokens");
    memset(s, 0, sizeof *s);
    const int64_t need = (len - 1 + 1 + ps - 1) / ps;
    if (grow(e->target_pages, &s->target_blocks, &s->n_target_blocks, need))
        return set_err("alloc target prefill pages");
    if (grow(e->draft_pages, &s->draft_blocks, &s->n_draft_blocks, need))
        return set_err("alloc draft prefill pages");
    s->kv_len = len - 1;
    s->last_token = prompt[len - 1];
    push_tokens(s, prompt, len);
    return 0;
}

int vxo_spec_step(vxo_spec *e, vxo_spec_state *st, int64_t n, int64_t d, int64_t eos,
                  int32_t *accepted, uint32_t *committed, int32_t *stop, uint32_t *tr_cand,
                  float *tr_logits) {
    if (d == 0) return set_err("draft_k must be >= 1");
    const int64_t ps = e->target_pages->page_size;
    if (e->draft_pages->page_size != ps) return set_err("draft page_size != target page_size");
    const int64_t V = e->target->cfg.vocab;
    for (int64_t b = 0; b < n; b++) {
        if (grow(e->target_pages, &st[b].target_blocks, &st[b].n_target_blocks,
                 (st[b].kv_len + d + 1 + ps - 1) / ps))
            return set_err("grow target block table");
        if (grow(e->draft_pages, &st[b].draft_blocks, &st[b].n_draft_blocks,
                 (st[b].kv_len + d + ps - 1) / ps))
            return set_err("grow draft block table");
    }
    const int stochastic = e->temperature > 0.0f;
    const float inv_t = stochastic ? 1.0f / e->temperature : 1.0f;
    uint32_t *cand = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)(n * d));
    float *dlog = (float *)malloc(sizeof(float) * (size_t)(n * d * V));
    float *tlog = (float *)malloc(sizeof(float) * (size_t)(n * (d + 1) * V));
    float *uni = (float *)malloc(sizeof(float) * (size_t)(n * (d + 1) * 4));
    uint32_t *ids = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)(n * (d + 1)));
    vxo_seq *sq = (vxo_seq *)malloc(sizeof(vxo_seq) * (size_t)n);
    int rc = 0;
    for (int64_t b = 0; b < n; b++) {
        vxo_spec_uniforms(e->sample_seed, st[b].stream_id, st[b].round, 1, d, uni + b * (d + 1) * 4);
    }
    /* draft phase: feed [last, c0 .. c_{D-2}] one token at a time */
    for (int64_t i = 0; i < d && rc == 0; i++) {
        for (int64_t b = 0; b < n; b++) {
            ids[b] = i == 0 ? st[b].last_token : cand[b * d + i - 1];
            sq[b] = (vxo_seq){1, st[b].kv_len + i, st[b].draft_blocks, st[b].n_draft_blocks};
        }
        float *row = (float *)malloc(sizeof(float) * (size_t)(n * V));
        rc = vxo_forward(e->draft, e->draft_pages, ids, sq, n, 0, NULL, row);
        for (int64_t b = 0; b < n && rc == 0; b++) {
            memcpy(dlog + (b * d + i) * V, row + b * V, sizeof(float) * (size_t)V);
            if (!stochastic) {
                cand[b * d + i] = vxo_argmax(row + b * V, V);
            } else {
                float m, z;
                vxo_row_softmax_stats(row + b * V, V, inv_t, &m, &z);
                cand[b * d + i] = vxo_sample_residual(row + b * V, m, z, NULL, 0.0f, 1.0f, V, inv_t,
                                                      uni[(b * (d + 1) + i) * 4 + 0]);
            }
        }
        free(row);
    }
    /* verify: feed [last, c0 .. c_{D-1}] to the target */
    if (rc == 0) {
        for (int64_t b = 0; b < n; b++) {
            ids[b * (d + 1)] = st[b].last_token;
            memcpy(ids + b * (d + 1) + 1, cand + b * d, sizeof(uint32_t) * (size_t)d);
            sq[b] = (vxo_seq){d + 1, st[b].kv_len, st[b].target_blocks, st[b].n_target_blocks};
        }
        rc = vxo_forward(e->target, e->target_pages, ids, sq, n, 1, NULL, tlog);
    }
    if (rc == 0) {
        uint32_t *tok = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)(n * (d + 1)));
        if (!stochastic)
            vxo_accept_greedy(tlog, V, cand, n, d, accepted, tok);
        else
            vxo_accept_stochastic(tlog, dlog, cand, uni, n, d, V, inv_t, accepted, tok);
        for (int64_t b = 0; b < n; b++) {
            const int64_t a = accepted[b];
            memcpy(committed + b * (d + 1), tok + b * (d + 1), sizeof(uint32_t) * (size_t)(a + 1));
            if (e->fix_draft_hole && a == d) {
                /* opt-in: also feed c[D-1] so the draft KV has no unwritten slot */
                uint32_t id1 = cand[b * d + d - 1];
                vxo_seq s1 = {1, st[b].kv_len + d, st[b].draft_blocks, st[b].n_draft_blocks};
                if (grow(e->draft_pages, &st[b].draft_blocks, &st[b].n_draft_blocks,
                         (st[b].kv_len + d + 1 + ps - 1) / ps) == 0) {
                    s1.block_table = st[b].draft_blocks;
                    s1.n_blocks = st[b].n_draft_blocks;
                    float *row = (float *)malloc(sizeof(float) * (size_t)V);
                    rc = vxo_forward(e->draft, e->draft_pages, &id1, &s1, 1, 0, NULL, row);
                    free(row);
                }
            }
            st[b].kv_len += a + 1;
            st[b].last_token = tok[b * (d + 1) + a];
            push_tokens(&st[b], tok + b * (d + 1), a + 1);
            st[b].round++;
            int sp = 0;
            if (eos >= 0)
                for (int64_t i = 0; i <= a; i++)
                    if (tok[b * (d + 1) + i] == (uint32_t)eos) sp = 1;
            stop[b] = sp;
        }
        if (tr_cand) memcpy(tr_cand, cand, sizeof(uint32_t) * (size_t)(n * d));
        if (tr_logits) memcpy(tr_logits, tlog, sizeof(float) * (size_t)(n * (d + 1) * V));
        free(tok);
    }
    free(cand);
    free(dlog);
    free(tlog);
    free(uni);
    free(ids);
    free(sq);
    return rc;
}

void vxo_spec_free(vxo_spec *e, vxo_spec_state *s) {
    vxo_pages_free(e->target_pages, s->target_blocks, s->n_target_blocks);
    vxo_pages_free(e->draft_pages, s->draft_blocks, s->n_draft_blocks);
    free(s->target_blocks);
    free(s->draft_blocks);
    free(s->tokens);
    memset(s, 0, sizeof *s);
}
