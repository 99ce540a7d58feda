/*
 * skyla_oracle.c -- CPU restatement of the reference's f32 quantized weight path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path and the reported CPU baseline.
 * Nothing in the product library links, loads or calls this file.
 *
 * Each function cites the reference file:line it restates.  Operation order follows the
 * Rust exactly (no contraction, sequential reductions starting at -0.0 as core's
 * `impl Sum for f32` does), so on the same host the results are the reference's.
 */
#define _GNU_SOURCE
#include "skyla_oracle.h"

#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

static inline float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

/* IEEE-754 binary16 -> binary32, exact for every pattern.  NaNs keep their payload and
 * come back quiet, as half 2.7.1 f16::to_f32 does (quant.rs:14, 19, 52-53, 71). */
float sk_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    if (exp == 0x1fu) {
        if (man == 0) return bits_f32(sign | 0x7f800000u);
        return bits_f32(sign | 0x7fc00000u | (man << 13));
    }
    if (exp == 0) {
        if (man == 0) return bits_f32(sign);
        /* subnormal: man * 2^-24; normalise so the leading one becomes implicit */
        int e = -14;
        while ((man & 0x400u) == 0) {
            man <<= 1;
            e -= 1;
        }
        man &= 0x3ffu;
        return bits_f32(sign | ((uint32_t)(e + 127) << 23) | (man << 13));
    }
    return bits_f32(sign | ((exp - 15u + 127u) << 23) | (man << 13));
}

/* binary32 -> binary16 with round-to-nearest-even (half f16::from_f32, quant.rs:96). */
uint16_t sk_f32_to_f16(float f) {
    uint32_t x = f32_bits(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xffu) {
        if (man == 0) return sign | 0x7c00u;
        return sign | 0x7e00u | (uint16_t)(man >> 13);
    }
    int e = (int)exp - 127;
    if (e >= 16) return sign | 0x7c00u;
    if (e >= -14) {
        uint32_t hm = ((uint32_t)(e + 15) << 10) | (man >> 13);
        uint32_t rem = man & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) hm += 1; /* may carry to inf */
        return sign | (uint16_t)hm;
    }
    if (e < -25) return sign;
    uint32_t m = man | 0x800000u;
    uint32_t shift = (uint32_t)(-e - 1);
    uint32_t hm = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t halfway = 1u << (shift - 1u);
    if (rem > halfway || (rem == halfway && (hm & 1u))) hm += 1;
    return sign | (uint16_t)hm;
}

/* DType::block (skyla-gguf/src/lib.rs:33-43) */
int sk_block(uint32_t type, uint64_t *per_block, uint64_t *bytes) {
    uint64_t p, b;
    switch (type) {
    case SK_F32: p = 1; b = 4; break;
    case SK_F16: p = 1; b = 2; break;
    case SK_Q8_0: p = 32; b = 34; break;
    case SK_Q4K: p = 256; b = 144; break;
    case SK_Q6K: p = 256; b = 210; break;
    default: return SK_E_TYPE;
    }
    if (per_block) *per_block = p;
    if (bytes) *bytes = b;
    return SK_OK;
}

/* DType::row_bytes (skyla-gguf/src/lib.rs:45-53) */
int64_t sk_row_bytes(uint32_t type, uint64_t n) {
    uint64_t p, b;
    if (sk_block(type, &p, &b) != SK_OK) return SK_E_TYPE;
    if (n % p != 0) return SK_E_ROW;
    return (int64_t)(n / p * b);
}

static inline uint16_t le16(const uint8_t *b) { return (uint16_t)(b[0] | (b[1] << 8)); }

/* quant.rs:40-49 */
void sk_q4k_scale_min(uint32_t j, const uint8_t *s, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0xf) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* quant.rs:51-68 */
static void dequantize_q4k(const uint8_t *b, float *out) {
    float d = sk_f16_to_f32(le16(b));
    float dmin = sk_f16_to_f32(le16(b + 2));
    const uint8_t *scales = b + 4;
    const uint8_t *qs = b + 16;
    for (int chunk = 0; chunk < 4; chunk++) {
        const uint8_t *q = qs + chunk * 32;
        uint8_t sc0, m0, sc1, m1;
        sk_q4k_scale_min((uint32_t)(chunk * 2), scales, &sc0, &m0);
        sk_q4k_scale_min((uint32_t)(chunk * 2 + 1), scales, &sc1, &m1);
        float d0 = d * (float)sc0, min0 = dmin * (float)m0;
        float d1 = d * (float)sc1, min1 = dmin * (float)m1;
        float *o = out + chunk * 64;
        for (int l = 0; l < 32; l++) {
            o[l] = d0 * (float)(q[l] & 0xf) - min0;
            o[l + 32] = d1 * (float)(q[l] >> 4) - min1;
        }
    }
}

/* quant.rs:70-89 */
static void dequantize_q6k(const uint8_t *b, float *out) {
    float d = sk_f16_to_f32(le16(b + 208));
    for (int half = 0; half < 2; half++) {
        const uint8_t *ql = b + half * 64;
        const uint8_t *qh = b + 128 + half * 32;
        const int8_t *sc = (const int8_t *)(b + 192 + half * 8);
        float *o = out + half * 128;
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int q1 = (int)((ql[l] & 0xf) | ((qh[l] & 3) << 4)) - 32;
            int q2 = (int)((ql[l + 32] & 0xf) | (((qh[l] >> 2) & 3) << 4)) - 32;
            int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            o[l] = d * (float)sc[is] * (float)q1;
            o[l + 32] = d * (float)sc[is + 2] * (float)q2;
            o[l + 64] = d * (float)sc[is + 4] * (float)q3;
            o[l + 96] = d * (float)sc[is + 6] * (float)q4;
        }
    }
}

/* quant.rs:5-38.  Like the Rust zip over chunks, only whole blocks that fit both the
 * source and the output are converted. */
int sk_dequantize(uint32_t type, const uint8_t *src, uint64_t src_len, float *out, uint64_t out_len) {
    uint64_t per, bytes;
    if (sk_block(type, &per, &bytes) != SK_OK) return SK_E_TYPE;
    uint64_t blocks = src_len / bytes;
    uint64_t out_blocks = type == SK_F32 || type == SK_F16 ? out_len : out_len / per;
    if (type == SK_Q8_0 || type == SK_Q4K || type == SK_Q6K) {
        /* chunks_mut(per) also yields a final partial chunk; the reference writes
         * into it only for Q8_0 (zip stops at the shorter side) */
        uint64_t partial = out_len % per;
        if (partial && type == SK_Q8_0) out_blocks += 1;
    }
    uint64_t n = blocks < out_blocks ? blocks : out_blocks;
    for (uint64_t i = 0; i < n; i++) {
        const uint8_t *b = src + i * bytes;
        switch (type) {
        case SK_F32: {
            out[i] = bits_f32((uint32_t)b[0] | ((uint32_t)b[1] << 8) | ((uint32_t)b[2] << 16) |
                              ((uint32_t)b[3] << 24));
            break;
        }
        case SK_F16: out[i] = sk_f16_to_f32(le16(b)); break;
        case SK_Q8_0: {
            float d = sk_f16_to_f32(le16(b));
            uint64_t len = out_len - i * 32 < 32 ? out_len - i * 32 : 32;
            for (uint64_t k = 0; k < len; k++) out[i * 32 + k] = d * (float)(int8_t)b[2 + k];
            break;
        }
        case SK_Q4K: dequantize_q4k(b, out + i * 256); break;
        case SK_Q6K: dequantize_q6k(b, out + i * 256); break;
        }
    }
    return SK_OK;
}

/* quant.rs:91-101 */
void sk_quantize_q8_0(const float *src, uint64_t n, uint8_t *out) {
    for (uint64_t blk = 0; blk * 32 < n; blk++) {
        const float *x = src + blk * 32;
        uint64_t len = n - blk * 32 < 32 ? n - blk * 32 : 32;
        uint8_t *b = out + blk * 34;
        float amax = 0.0f;
        for (uint64_t i = 0; i < len; i++) amax = fmaxf(amax, fabsf(x[i]));
        float d = amax / 127.0f;
        float inv = d > 0.0f ? 1.0f / d : 0.0f;
        uint16_t h = sk_f32_to_f16(d);
        b[0] = (uint8_t)h;
        b[1] = (uint8_t)(h >> 8);
        for (uint64_t i = 0; i < len; i++) {
            float v = roundf(x[i] * inv); /* f32::round: half away from zero */
            if (v != v) v = 0.0f;          /* `as i8` saturates NaN to 0 */
            if (v < -127.0f) v = -127.0f;
            if (v > 127.0f) v = 127.0f;
            b[2 + i] = (uint8_t)(int8_t)v;
        }
    }
}

/* ops.rs:32-34 dot: a sequential fold from -0.0 */
float sk_dot(const float *a, const float *b, uint64_t n) {
    float s = -0.0f;
    for (uint64_t i = 0; i < n; i++) s += a[i] * b[i];
    return s;
}

/* ops.rs:1-16 rmsnorm + inv_rms */
void sk_rmsnorm(const float *x, const float *w, uint64_t n, float eps, float *out) {
    float ss = -0.0f;
    for (uint64_t i = 0; i < n; i++) ss += x[i] * x[i];
    float ms = ss / (float)n;
    float r = 1.0f / sqrtf(ms + eps);
    for (uint64_t i = 0; i < n; i++) out[i] = x[i] * r * w[i];
}

/* ops.rs:8-16 rmsnorm_inplace: x *= r * w (note the grouping, unlike rmsnorm) */
void sk_rmsnorm_inplace(float *x, const float *w, uint64_t n, float eps) {
    float ss = -0.0f;
    for (uint64_t i = 0; i < n; i++) ss += x[i] * x[i];
    float ms = ss / (float)n;
    float r = 1.0f / sqrtf(ms + eps);
    for (uint64_t i = 0; i < n; i++) x[i] *= r * w[i];
}

/* rope.rs:36-40 frequencies without scaling (no YaRN): theta^(-2i / d), i < d / 2 */
void sk_rope_freqs(uint64_t head_dim, float theta, float *out) {
    float d = (float)head_dim;
    for (uint64_t i = 0; i < head_dim / 2; i++) out[i] = powf(theta, -2.0f * (float)i / d);
}

/* rope.rs:32-34 corr_dim: the dimension whose wavelength makes n_rot turns over
 * original_ctx positions, n_dims * ln(original_ctx / (n_rot * 2 pi)) / (2 ln base) */
static float corr_dim(float n_dims, float original_ctx, float n_rot, float base) {
    return n_dims * logf(original_ctx / (n_rot * 2.0f * (float)M_PI)) / (2.0f * logf(base));
}

/* rope.rs:36-58 frequencies with YaRN scaling (factor, original_ctx, attn_factor): each
 * base frequency f_i times freq_scale (1 - mix) + mix, where mix ramps from 1 below the
 * dimension of beta_fast = 32 turns to 0 above that of beta_slow = 1 turn and freq_scale =
 * 1 / factor; returns the magnitude scale attn_factor * (1 + 0.1 ln(1 / freq_scale)). */
float sk_rope_freqs_yarn(uint64_t head_dim, float theta, float factor, float original_ctx, float attn_factor,
                         float *out) {
    const float d = (float)head_dim;
    const float freq_scale = 1.0f / factor;
    const float low = fmaxf(floorf(corr_dim(d, original_ctx, 32.0f, theta)), 0.0f);
    const float high = fminf(ceilf(corr_dim(d, original_ctx, 1.0f, theta)), d - 1.0f);
    for (uint64_t i = 0; i < head_dim / 2; i++) {
        const float f = powf(theta, -2.0f * (float)i / d);
        const float y = ((float)i - low) / fmaxf(high - low, 0.001f);
        const float mix = 1.0f - fminf(fmaxf(y, 0.0f), 1.0f);
        out[i] = f * (freq_scale * (1.0f - mix) + mix);
    }
    return attn_factor * (1.0f + 0.1f * logf(1.0f / freq_scale));
}

/* rope.rs:60-68 rope_neox over x[0..n): pairs (i, i + n/2) rotated by pos * freqs[i] */
void sk_rope_neox(float *x, uint64_t n, uint64_t pos, const float *freqs, float mscale) {
    uint64_t half = n / 2;
    for (uint64_t i = 0; i < half; i++) {
        float ang = (float)pos * freqs[i];
        float sn = sinf(ang) * mscale, cs = cosf(ang) * mscale;
        float a = x[i], b = x[i + half];
        x[i] = a * cs - b * sn;
        x[i + half] = a * sn + b * cs;
    }
}

/* model.rs:150-169, the attention of every head over the f32 cache of n_pos positions
 * (no output gate): scores = q.k * (1 / sqrt(hd)), softmax, o = sum_p w_p v_p in position
 * order from 0.  scores holds n_pos floats of scratch. */
void sk_attention(const float *q, const float *k_cache, const float *v_cache, uint64_t n_pos,
                  uint64_t n_head, uint64_t n_head_kv, uint64_t hd, float *scores, float *out) {
    uint64_t kv_dim = n_head_kv * hd, n_rep = n_head / n_head_kv;
    float scale = 1.0f / sqrtf((float)hd);
    for (uint64_t h = 0; h < n_head; h++) {
        uint64_t base = (h / n_rep) * hd;
        const float *qh = q + h * hd;
        for (uint64_t p = 0; p < n_pos; p++) scores[p] = sk_dot(qh, k_cache + p * kv_dim + base, hd) * scale;
        sk_softmax(scores, n_pos);
        float *oh = out + h * hd;
        for (uint64_t d = 0; d < hd; d++) oh[d] = 0.0f;
        for (uint64_t p = 0; p < n_pos; p++) {
            const float *vp = v_cache + p * kv_dim + base;
            float w = scores[p];
            for (uint64_t d = 0; d < hd; d++) oh[d] += w * vp[d];
        }
    }
}

/* ops.rs:18-26 */
void sk_softmax(float *x, uint64_t n) {
    float max = -INFINITY;
    for (uint64_t i = 0; i < n; i++) max = fmaxf(max, x[i]); /* f32::max ignores NaN */
    float sum = 0.0f;
    for (uint64_t i = 0; i < n; i++) {
        x[i] = expf(x[i] - max);
        sum += x[i];
    }
    for (uint64_t i = 0; i < n; i++) x[i] /= sum;
}

/* ops.rs:28-30 */
float sk_silu(float x) { return x / (1.0f + expf(-x)); }

/* f32::total_cmp key (ops.rs:36-41 argmax, ffn.rs:32 route sort) */
static inline int32_t total_key(float f) {
    int32_t i = (int32_t)f32_bits(f);
    i ^= (int32_t)(((uint32_t)(i >> 31)) >> 1);
    return i;
}

/* ops.rs:36-41: Iterator::max_by keeps the LAST of equal maxima. */
uint32_t sk_argmax(const float *x, uint64_t n) {
    if (n == 0) return 0;
    uint64_t best = 0;
    for (uint64_t i = 1; i < n; i++)
        if (total_key(x[i]) >= total_key(x[best])) best = i;
    return (uint32_t)best;
}

/* ---- Matrix::matvec (matrix.rs:43-58) ---- */

uint32_t sk_available_parallelism(void) {
    cpu_set_t set;
    if (sched_getaffinity(0, sizeof(set), &set) == 0) {
        int c = CPU_COUNT(&set);
        if (c > 0) return (uint32_t)c;
    }
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (uint32_t)n : 8u; /* map_or(8, ..) */
}

struct mv_job {
    uint32_t type;
    const uint8_t *data;
    uint64_t n_in, row_bytes, first, count;
    const float *x;
    float *y;
    int status;
};

static void *mv_worker(void *arg) {
    struct mv_job *j = (struct mv_job *)arg;
    float *row = (float *)malloc(j->n_in * sizeof(float));
    if (!row) {
        j->status = SK_E_THREAD;
        return NULL;
    }
    for (uint64_t i = 0; i < j->count; i++) {
        uint64_t r = j->first + i;
        /* Matrix::row (matrix.rs:38-41) then the sequential dot */
        sk_dequantize(j->type, j->data + r * j->row_bytes, j->row_bytes, row, j->n_in);
        float s = -0.0f;
        for (uint64_t k = 0; k < j->n_in; k++) s += row[k] * j->x[k];
        j->y[i] = s;
    }
    free(row);
    j->status = SK_OK;
    return NULL;
}

int sk_matvec(uint32_t type, const uint8_t *data, uint64_t n_in, uint64_t n_out,
              const float *x, float *y, uint32_t threads) {
    int64_t rb = sk_row_bytes(type, n_in);
    if (rb < 0) return (int)rb;
    if (n_out == 0) return SK_OK;
    uint64_t t = threads ? threads : sk_available_parallelism();
    uint64_t per = (n_out + t - 1) / t; /* n_out.div_ceil(threads) */
    uint64_t n_jobs = (n_out + per - 1) / per;
    struct mv_job *jobs = (struct mv_job *)calloc(n_jobs, sizeof(struct mv_job));
    pthread_t *tids = (pthread_t *)calloc(n_jobs, sizeof(pthread_t));
    if (!jobs || !tids) {
        free(jobs);
        free(tids);
        return SK_E_THREAD;
    }
    int status = SK_OK;
    uint64_t started = 0;
    for (uint64_t k = 0; k < n_jobs; k++) {
        uint64_t first = k * per;
        uint64_t count = n_out - first < per ? n_out - first : per;
        jobs[k] = (struct mv_job){type, data, n_in, (uint64_t)rb, first, count, x, y + first, SK_OK};
        if (n_jobs == 1) {
            mv_worker(&jobs[k]);
        } else if (pthread_create(&tids[k], NULL, mv_worker, &jobs[k]) != 0) {
            status = SK_E_THREAD;
            break;
        }
        started++;
    }
    if (n_jobs > 1)
        for (uint64_t k = 0; k < started; k++) pthread_join(tids[k], NULL);
    for (uint64_t k = 0; k < started; k++)
        if (jobs[k].status != SK_OK) status = jobs[k].status;
    free(jobs);
    free(tids);
    return status;
}

int sk_matmul(uint32_t type, const uint8_t *data, uint64_t n_in, uint64_t n_out, uint64_t n_tok,
              const float *x, uint64_t x_stride, float *y, uint64_t y_stride, uint32_t threads) {
    for (uint64_t t = 0; t < n_tok; t++) {
        int s = sk_matvec(type, data, n_in, n_out, x + t * x_stride, y + t * y_stride, threads);
        if (s != SK_OK) return s;
    }
    return SK_OK;
}

/* ---- ffn.rs ---- */

/* ffn.rs:30-37: logits by sequential dot, stable sort descending by total_cmp (equal
 * logits keep index order), truncate to `used`, softmax. */
int sk_route(const float *router, const float *n, uint64_t n_embd, uint64_t n_expert,
             uint64_t used, uint32_t *ids, float *weights) {
    if (used > n_expert) used = n_expert; /* Vec::truncate never grows */
    float *logit = (float *)malloc(n_expert * sizeof(float));
    uint32_t *order = (uint32_t *)malloc(n_expert * sizeof(uint32_t));
    if (!logit || !order) {
        free(logit);
        free(order);
        return SK_E_THREAD;
    }
    for (uint64_t e = 0; e < n_expert; e++) {
        logit[e] = sk_dot(router + e * n_embd, n, n_embd);
        order[e] = (uint32_t)e;
    }
    /* insertion sort is stable: an element moves left only past strictly smaller keys */
    for (uint64_t i = 1; i < n_expert; i++) {
        uint32_t cur = order[i];
        int32_t key = total_key(logit[cur]);
        uint64_t j = i;
        while (j > 0 && total_key(logit[order[j - 1]]) < key) {
            order[j] = order[j - 1];
            j--;
        }
        order[j] = cur;
    }
    for (uint64_t k = 0; k < used; k++) {
        ids[k] = order[k];
        weights[k] = logit[order[k]];
    }
    sk_softmax(weights, used);
    free(logit);
    free(order);
    return SK_OK;
}

/* ffn.rs:21-28 */
int sk_swiglu(uint32_t gate_type, const uint8_t *gate, uint32_t up_type, const uint8_t *up,
              uint32_t down_type, const uint8_t *down, uint64_t n_embd, uint64_t n_ff,
              const float *n, float *out, uint32_t threads) {
    float *g = (float *)malloc(n_ff * sizeof(float));
    float *u = (float *)malloc(n_ff * sizeof(float));
    int s = (!g || !u) ? SK_E_THREAD : SK_OK;
    if (s == SK_OK) s = sk_matvec(gate_type, gate, n_embd, n_ff, n, g, threads);
    if (s == SK_OK) s = sk_matvec(up_type, up, n_embd, n_ff, n, u, threads);
    if (s == SK_OK) {
        for (uint64_t i = 0; i < n_ff; i++) g[i] = sk_silu(g[i]) * u[i];
        s = sk_matvec(down_type, down, n_ff, n_embd, g, out, threads);
    }
    free(g);
    free(u);
    return s;
}

/* ffn.rs:58-76 (Moe arm); Matrix::expert slices e * n_out * row_bytes (matrix.rs:30-36) */
int sk_moe_forward(const float *router, uint32_t gate_type, const uint8_t *gate_exps,
                   uint32_t up_type, const uint8_t *up_exps, uint32_t down_type,
                   const uint8_t *down_exps, uint64_t n_embd, uint64_t n_ff, uint64_t n_expert,
                   uint64_t used, const float *n, float *out, uint32_t *ids, float *weights,
                   uint32_t threads) {
    int64_t rb_g = sk_row_bytes(gate_type, n_embd), rb_u = sk_row_bytes(up_type, n_embd);
    int64_t rb_d = sk_row_bytes(down_type, n_ff);
    if (rb_g < 0) return (int)rb_g;
    if (rb_u < 0) return (int)rb_u;
    if (rb_d < 0) return (int)rb_d;
    if (used > n_expert) used = n_expert;
    uint32_t *rid = (uint32_t *)malloc((used ? used : 1) * sizeof(uint32_t));
    float *rw = (float *)malloc((used ? used : 1) * sizeof(float));
    float *y = (float *)malloc(n_embd * sizeof(float));
    int s = (!rid || !rw || !y) ? SK_E_THREAD : SK_OK;
    if (s == SK_OK) s = sk_route(router, n, n_embd, n_expert, used, rid, rw);
    if (s == SK_OK) {
        for (uint64_t i = 0; i < n_embd; i++) out[i] = 0.0f;
        for (uint64_t k = 0; k < used && s == SK_OK; k++) {
            uint64_t e = rid[k];
            s = sk_swiglu(gate_type, gate_exps + e * n_ff * (uint64_t)rb_g, up_type,
                          up_exps + e * n_ff * (uint64_t)rb_u, down_type,
                          down_exps + e * n_embd * (uint64_t)rb_d, n_embd, n_ff, n, y, threads);
            for (uint64_t i = 0; i < n_embd; i++) out[i] += rw[k] * y[i];
        }
        if (ids)
            for (uint64_t k = 0; k < used; k++) ids[k] = rid[k];
        if (weights)
            for (uint64_t k = 0; k < used; k++) weights[k] = rw[k];
    }
    free(rid);
    free(rw);
    free(y);
    return s;
}

/* moe_sort.comp:21-55: per-expert counts, exclusive scan into (count, start), and a
 * stable rank so list[start[e] + rank] = slot. */
int sk_moe_sort(const uint32_t *ids, uint64_t n_slots, uint32_t n_expert, uint32_t *table,
                uint32_t *list) {
    uint32_t *count = (uint32_t *)calloc(n_expert ? n_expert : 1, sizeof(uint32_t));
    uint32_t *fill = (uint32_t *)calloc(n_expert ? n_expert : 1, sizeof(uint32_t));
    if (!count || !fill) {
        free(count);
        free(fill);
        return SK_E_THREAD;
    }
    for (uint64_t i = 0; i < n_slots; i++) {
        if (ids[i] >= n_expert) {
            free(count);
            free(fill);
            return SK_E_SIZE;
        }
        count[ids[i]]++;
    }
    uint32_t s = 0;
    for (uint32_t e = 0; e < n_expert; e++) {
        table[2 * e] = count[e];
        table[2 * e + 1] = s;
        fill[e] = s;
        s += count[e];
    }
    for (uint64_t i = 0; i < n_slots; i++) list[fill[ids[i]]++] = (uint32_t)i;
    free(count);
    free(fill);
    return SK_OK;
}
