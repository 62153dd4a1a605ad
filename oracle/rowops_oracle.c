/*
 * CPU oracle for the fused row ops — TEST INFRASTRUCTURE ONLY (see rowops_oracle.h).
 *
 * Built with -ffp-contract=off so every fp32 expression is rounded exactly as written: the
 * reference's rounding points are restated operation by operation, while reductions and
 * transcendentals are evaluated more accurately (double) than the GPU does, so the oracle is the
 * "reference semantics with exact arithmetic" the tolerances are measured from.
 */
#include "rowops_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

int oracle_mutation = ORM_NONE;

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------------------------------ */
/* Conversions.  f32 -> f16 follows IEEE 754 binary16 RNE (the semantics of __float2half_rn used
 * at kernels/norm.cu:75-83 and kernels/rope.cu:168-169); f32 -> bf16 is RNE as torch rounds it. */

uint16_t oracle_f32_to_f16(float f)
{
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);          /* >= 65520 rounds to inf */
    if (ax < 0x38800000u)                                               /* below 2^-14: subnormal */
    {
        if (ax <= 0x33000000u) return (uint16_t)sign;                   /* <= 2^-25 rounds to 0 */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e;                                      /* 14 .. 24 */
        uint32_t r = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = (ax - 0x38000000u) >> 13;
    uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return (uint16_t)(sign | r);
}

float oracle_f16_to_f32(uint16_t h)
{
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t m = (uint32_t)h & 0x3ffu;
    if (e == 0)
    {
        float v = (float)m * 0x1p-24f;
        return u2f(f2u(v) | sign);
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t oracle_f32_to_bf16(float f)
{
    uint32_t x = f2u(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x0040u);
    uint32_t lsb = (x >> 16) & 1u;
    x += 0x7fffu + lsb;
    return (uint16_t)(x >> 16);
}

float oracle_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

static double round_fmt(double v, int mant_bits, int emin, double maxv)
{
    if (v != v || isinf(v) || v == 0.0) return v;
    int e;
    frexp(v, &e);
    int lead = e - 1;
    if (lead < emin) lead = emin;
    double q = ldexp(1.0, lead - (mant_bits - 1));
    double r = nearbyint(v / q) * q;
    if (fabs(r) > maxv) r = copysign(INFINITY, v);
    return r;
}

double oracle_round(double v, int dtype)
{
    switch (dtype)
    {
        case OR_F16:  return round_fmt(v, 11, -14, 65504.0);
        case OR_BF16: return round_fmt(v, 8, -126, 0x1.fep127);
        default:      return (double)(float)v;
    }
}

void oracle_f32_to_f16_array(const float* in, uint16_t* out, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_f32_to_f16(in[i]);
}

void oracle_f32_to_bf16_array(const float* in, uint16_t* out, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_f32_to_bf16(in[i]);
}

static inline float ld(const void* p, int dt, int64_t i)
{
    switch (dt)
    {
        case OR_F16:  return oracle_f16_to_f32(((const uint16_t*)p)[i]);
        case OR_BF16: return oracle_bf16_to_f32(((const uint16_t*)p)[i]);
        default:      return ((const float*)p)[i];
    }
}

/* Store an fp32 value, rounded once (RNE) to dt. */
static inline void st(void* p, int dt, int64_t i, float v)
{
    switch (dt)
    {
        case OR_F16:  ((uint16_t*)p)[i] = oracle_f32_to_f16(v); break;
        case OR_BF16: ((uint16_t*)p)[i] = oracle_f32_to_bf16(v); break;
        default:      ((float*)p)[i] = v; break;
    }
}

/* Value of v after rounding to dt (what st() followed by ld() yields). */
static inline float rnd(float v, int dt)
{
    switch (dt)
    {
        case OR_F16:  return oracle_f16_to_f32(oracle_f32_to_f16(v));
        case OR_BF16: return oracle_bf16_to_f32(oracle_f32_to_bf16(v));
        default:      return v;
    }
}

/* CLAMP_FP16 = fmaxf(-65504, fminf(x, 65504)) (kernels/util.cuh:69-70): +-inf -> +-65504, NaN -> 65504 */
static inline float clamp_f16(float v) { return fmaxf(-65504.0f, fminf(v, 65504.0f)); }

static int nthr(int n) { return n > 0 ? n : 1; }

static int fdtype(int dt) { return dt == OR_F32 || dt == OR_F16 || dt == OR_BF16; }

/* ------------------------------------------------------------------------------------------ */
/* RMSNorm, plain and residual-fused.
 * Follows rms_norm_kernel (kernels/norm.cu:160-304):
 *   - f16 x clamped on read (read_half4<true>, norm.cu:42-58, used by read_in at 192-196);
 *   - RES_IN: r <- round_r(x + r) in place, then the norm reads the rounded sum (add_resid_in,
 *     norm.cu:198-223);
 *   - sum of squares (norm.cu:101-108, reduced 140-151; here in double, rounded once to fp32);
 *   - rmf = rsqrt(sum / dim + eps) * constant_scale (norm.cu:273, 288), evaluated as an IEEE fp32
 *     sqrt and an IEEE fp32 division (the reference's rsqrtf is an approximation of the same);
 *   - y = (x * (w + constant_bias)) * rmf in fp32 (apply4, norm.cu:110-116, bias 232-239), or
 *     x * rmf without a weight (apply4_nw, 118-124), rounded once to y's dtype (write_half4, 75-83). */
static void rms_row(const float* h, const float* wf, void* y, int yt, int64_t yoff, int64_t dim,
                    float eps, float cs)
{
    double s = 0.0;
    for (int64_t j = 0; j < dim; ++j) s += (double)h[j] * (double)h[j];
    float sf = (float)s;
    int64_t d = oracle_mutation == ORM_RMS_DIM_OFF ? dim - 1 : dim;
    float mean = sf / (float)d;
    float t = oracle_mutation == ORM_RMS_NO_EPS ? mean : mean + eps;
    float rmf = 1.0f / sqrtf(t);
    rmf = rmf * cs;
    for (int64_t j = 0; j < dim; ++j)
    {
        float v = wf ? (h[j] * wf[j]) * rmf : h[j] * rmf;
        st(y, yt, yoff + j, v);
    }
}

static float* weight_f32(const void* w, int wt, int64_t dim, float cb)
{
    if (!w) return NULL;
    float* wf = (float*)malloc((size_t)dim * sizeof(float));
    for (int64_t j = 0; j < dim; ++j)
    {
        float v = ld(w, wt, j);
        if (cb != 0.0f && oracle_mutation != ORM_RMS_NO_BIAS) v = v + cb;
        wf[j] = v;
    }
    return wf;
}

int oracle_rms_norm(const void* x, int xt, int64_t ldx, const void* w, int wt, void* y, int yt, int64_t ldy,
                    void* r, int rt, int64_t ldr, int64_t rows, int64_t dim,
                    float eps, float cb, float cs, int nthreads)
{
    if (!x || !y || dim <= 0 || rows < 0) return -1;
    if (!fdtype(xt) || !fdtype(yt) || (w && !fdtype(wt)) || (r && !fdtype(rt))) return -2;
    float* wf = weight_f32(w, wt, dim, cb);

    #pragma omp parallel num_threads(nthr(nthreads))
    {
        float* h = (float*)malloc((size_t)dim * sizeof(float));
        #pragma omp for schedule(static)
        for (int64_t i = 0; i < rows; ++i)
        {
            for (int64_t j = 0; j < dim; ++j)
            {
                float xv = ld(x, xt, i * ldx + j);
                if (xt == OR_F16 && oracle_mutation != ORM_RMS_NO_CLAMP) xv = clamp_f16(xv);
                if (r)
                {
                    float hv = xv + ld(r, rt, i * ldr + j);
                    st(r, rt, i * ldr + j, hv);
                    if (oracle_mutation != ORM_RES_NO_ROUND) hv = rnd(hv, rt);
                    xv = hv;
                }
                h[j] = xv;
            }
            rms_row(h, wf, y, yt, i * ldy, dim, eps, cs);
        }
        free(h);
    }
    free(wf);
    return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* Gated activations, the reference's fp32 path (act_mul_kernel_f, kernels/activation_kernels.cuh:
 * 189-252) applied to upcast inputs:
 *   silu(x) = x / (1 + exp(-x))                    (activation_kernels.cuh:34-39)
 *   gelu(x) = 0.5 x (1 + tanh(sqrt(2/pi)(x + 0.044715 x^3)))   (activation_kernels.cuh:52-58,
 *             tanh-form GELU of Hendrycks & Gimpel); evaluated in double through the identity
 *             0.5 (1 + tanh(u)) = 1 / (1 + exp(-2u)), which has no cancellation for x << 0;
 *   act_limit: y clamped to [-L, L], act clamped from above (activation_kernels.cuh:237-245);
 *   product in fp32, one RNE to z's dtype, f16 z clamped to +-65504 (clamp_half2_to_finite,
 *   activation_kernels.cuh:2-7, 249-251; __hmin2/__hmax2 return the non-NaN operand). */
static double act_d(int act, double x)
{
    if (act == OR_ACT_SILU)
    {
        double e = oracle_mutation == ORM_SILU_SIGN ? exp(x) : exp(-x);
        return x / (1.0 + e);
    }
    if (act == OR_ACT_SIGMOID)   /* mul_sigmoid_ (activation.cu:532-568), _sigmoid_f (norm.cu:133-136) */
        return 1.0 / (1.0 + (oracle_mutation == ORM_SIGMOID_SIGN ? exp(x) : exp(-x)));
    const double c = 0.79788456080286535588;   /* sqrt(2/pi) */
    double cubic = oracle_mutation == ORM_GELU_NO_CUBIC ? 0.0 : 0.044715 * x * x * x;
    double u = c * (x + cubic);
    return x / (1.0 + exp(-2.0 * u));
}

int oracle_act_mul(int act, const void* x, const void* y, int it, void* z, int zt,
                   int64_t rows, int64_t cols, int64_t ldx, int64_t ldy, int64_t ldz,
                   float limit, int nthreads)
{
    if (!x || !y || !z || rows < 0 || cols < 0) return -1;
    if (!fdtype(it) || !fdtype(zt)) return -2;
    if (act != OR_ACT_SILU && act != OR_ACT_GELU && act != OR_ACT_SIGMOID) return -1;

    #pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int64_t i = 0; i < rows; ++i)
    {
        for (int64_t j = 0; j < cols; ++j)
        {
            float a = (float)act_d(act, (double)ld(x, it, i * ldx + j));
            float u = ld(y, it, i * ldy + j);
            if (limit != 0.0f)
            {
                if (oracle_mutation != ORM_ACT_NO_LIMIT_Y)
                {
                    if (u < -limit) u = -limit;
                    if (u > limit) u = limit;
                }
                if (a > limit) a = limit;
            }
            float p = a * u;
            if (zt == OR_F16) p = clamp_f16(p);
            st(z, zt, i * ldz + j, p);
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* Head RMSNorm + rotary embedding, following rope_kernel (kernels/rope.cu:16-255):
 *   pos = position + s | positions[b] + s | position_ids[b*seq + s]             (rope.cu:55-67)
 *   head norm (rope.cu:188-233), applied iff q_norm is given (rope.cu:250):
 *     sum of squares over the head (double here; the reference's reduction at rope.cu:196-204
 *     races on a shared slot, the intended full sum is used), rmf = 1 / sqrtf(sum/hd + eps),
 *     f16 weight with f16 I/O: out = h(h(w + h(cb)) * h(v * rmf)), two half roundings
 *       (rope.cu:222-229; half add/mul are correctly rounded);
 *     otherwise: out = io(fl32(fl32(v * rmf) * fl32(w + cb)))           (rope.cu:212-221);
 *   rotary (rope.cu:69-85, 152-185) on the io-rounded normed head:
 *     angle = fl32(inv_freq[t] * fl32(pos)); c = fl32(cos(angle)) * attn_factor, s likewise;
 *     NeoX pairs (t, t + R/2), GPT-J pairs (2t, 2t + 1), t < R/2;
 *     r1 = io(v1 c - v2 s), r2 = io(v2 c + v1 s) in fp32; dims >= R pass through. */
static void head_norm(float* v, int dt, int hd, const float* wf, const uint16_t* wh16, float eps)
{
    if (!wf && !wh16) return;
    double s = 0.0;
    for (int d = 0; d < hd; ++d) s += (double)v[d] * (double)v[d];
    float sf = (float)s;
    float rmf = 1.0f / sqrtf(sf / (float)hd + eps);
    for (int d = 0; d < hd; ++d)
    {
        float n = v[d] * rmf;
        if (wh16)
        {
            float wv = oracle_f16_to_f32(wh16[d]);
            if (oracle_mutation == ORM_HEADNORM_1ROUND)
                v[d] = rnd(n * wv, dt);
            else
                v[d] = rnd(rnd(n, OR_F16) * wv, OR_F16);   /* exact product of two halves */
        }
        else
            v[d] = rnd(n * wf[d], dt);
    }
}

static void rotate_head(float* v, int dt, int R, const float* cosv, const float* sinv, int mode)
{
    for (int t = 0; t < R / 2; ++t)
    {
        int i1, i2;
        if (mode == OR_ROPE_NEOX && oracle_mutation != ORM_ROPE_NEOX_PAIR) { i1 = t; i2 = t + R / 2; }
        else { i1 = 2 * t; i2 = 2 * t + 1; }
        float c = cosv[t], s = sinv[t];
        float v1 = v[i1], v2 = v[i2];
        float r1 = oracle_mutation == ORM_ROPE_SIGN ? v1 * c + v2 * s : v1 * c - v2 * s;
        float r2 = v2 * c + v1 * s;
        v[i1] = rnd(r1, dt);
        v[i2] = rnd(r2, dt);
    }
}

static void rope_head(const void* in, void* out, int64_t off, int dt, int hd, int R,
                      const float* cosv, const float* sinv, const float* wf, const uint16_t* wh16,
                      float eps, int mode, float* v)
{
    for (int d = 0; d < hd; ++d) v[d] = ld(in, dt, off + d);
    int norm_after = oracle_mutation == ORM_ROPE_NORM_AFTER;
    if (!norm_after) head_norm(v, dt, hd, wf, wh16, eps);
    rotate_head(v, dt, R, cosv, sinv, mode);
    if (norm_after) head_norm(v, dt, hd, wf, wh16, eps);
    for (int d = 0; d < hd; ++d) st(out, dt, off + d, v[d]);
}

/* Shared by oracle_rope (angle = inv_freq[t] * pos) and oracle_rope_table (angle read from the
 * table row of the token's sequence at pos; a position outside [0, table_rows) sets *err and
 * rotates by angle 0). */
static int rope_impl(const void* q, void* out_q, int64_t q_tok_stride, int64_t q_head_stride, int hq,
                     const void* k, void* out_k, int64_t k_tok_stride, int64_t k_head_stride, int hk,
                     int dt, int64_t bsz, int64_t seq_len, int hd,
                     const float* inv_freq, const float* table, int64_t table_rows, int64_t table_bstride,
                     int32_t* err, int R,
                     int32_t position, const int32_t* positions, const int32_t* position_ids,
                     const void* q_norm, const void* k_norm, int nwt,
                     float eps, float cb, int mode, float attn_factor, int nthreads)
{
    if (!q || !out_q || !(inv_freq || table) || hd <= 0 || (hd & 1) || R < 2 || (R & 1) || R > hd) return -1;
    if (dt != OR_F16 && dt != OR_BF16) return -2;
    if (mode != OR_ROPE_GPTJ && mode != OR_ROPE_NEOX) return -1;
    if (k && !out_k) return -1;
    if (!k) hk = 0;
    if (positions && position_ids) return -1;
    int norm = q_norm != NULL;
    if (norm && k && !k_norm) return -1;
    if (norm && !fdtype(nwt)) return -2;

    /* norm weights: f16 weight + f16 io -> half path (weights pre-added in half) */
    int half_path = norm && nwt == OR_F16 && dt == OR_F16;
    float* wfq = NULL; float* wfk = NULL; uint16_t* whq = NULL; uint16_t* whk = NULL;
    if (norm)
    {
        const void* ws[2] = { q_norm, k_norm };
        for (int which = 0; which < 2; ++which)
        {
            if (!ws[which]) continue;
            if (half_path)
            {
                uint16_t* wh = (uint16_t*)malloc((size_t)hd * 2);
                double cbh = (double)oracle_f16_to_f32(oracle_f32_to_f16(cb));
                for (int d = 0; d < hd; ++d)
                {
                    double sum = (double)ld(ws[which], nwt, d) + cbh;      /* __hadd2 (rope.cu:226) */
                    wh[d] = oracle_f32_to_f16((float)oracle_round(sum, OR_F16));
                }
                if (which == 0) whq = wh; else whk = wh;
            }
            else
            {
                float* wf = (float*)malloc((size_t)hd * sizeof(float));
                for (int d = 0; d < hd; ++d) wf[d] = ld(ws[which], nwt, d) + cb;
                if (which == 0) wfq = wf; else wfk = wf;
            }
        }
    }

    int64_t tokens = bsz * seq_len;
    #pragma omp parallel num_threads(nthr(nthreads))
    {
        float* v = (float*)malloc((size_t)hd * sizeof(float));
        float* cosv = (float*)malloc((size_t)(R / 2) * sizeof(float));
        float* sinv = (float*)malloc((size_t)(R / 2) * sizeof(float));
        #pragma omp for schedule(static)
        for (int64_t tok = 0; tok < tokens; ++tok)
        {
            int64_t b = tok / seq_len, s = tok % seq_len;
            int32_t pos = (int32_t)(position + s);
            if (positions) pos = (int32_t)(positions[b] + s);
            else if (position_ids) pos = position_ids[tok];
            if (oracle_mutation == ORM_ROPE_POS_OFF) pos += 1;
            float pf = (float)pos;
            int64_t trow = -1;
            if (table)
            {
                const int32_t tp = oracle_mutation == ORM_TABLE_ROW_OFF ? pos + 1 : pos;
                if (tp >= 0 && tp < table_rows) trow = b * table_bstride + (int64_t)tp * (R / 2);
                else if (err)
                {
                    #pragma omp atomic write
                    *err = 1;
                }
            }
            for (int t = 0; t < R / 2; ++t)
            {
                float a = table ? (trow >= 0 ? table[trow + t] : 0.0f) : inv_freq[t] * pf;
                float c = (float)cos((double)a) * attn_factor;
                float sn = (float)sin((double)a) * attn_factor;
                if (oracle_mutation == ORM_ROPE_SWAP_SINCOS) { float tmp = c; c = sn; sn = tmp; }
                cosv[t] = c;
                sinv[t] = sn;
            }
            for (int h = 0; h < hq; ++h)
                rope_head(q, out_q, tok * q_tok_stride + h * q_head_stride, dt, hd, R, cosv, sinv,
                          wfq, whq, eps, mode, v);
            for (int h = 0; h < hk; ++h)
                rope_head(k, out_k, tok * k_tok_stride + h * k_head_stride, dt, hd, R, cosv, sinv,
                          wfk, whk, eps, mode, v);
        }
        free(v); free(cosv); free(sinv);
    }
    free(wfq); free(wfk); free(whq); free(whk);
    return 0;
}

int oracle_rope(const void* q, void* out_q, int64_t q_tok_stride, int64_t q_head_stride, int hq,
                const void* k, void* out_k, int64_t k_tok_stride, int64_t k_head_stride, int hk,
                int dt, int64_t bsz, int64_t seq_len, int hd,
                const float* inv_freq, int R,
                int32_t position, const int32_t* positions, const int32_t* position_ids,
                const void* q_norm, const void* k_norm, int nwt,
                float eps, float cb, int mode, float attn_factor, int nthreads)
{
    if (!inv_freq) return -1;
    return rope_impl(q, out_q, q_tok_stride, q_head_stride, hq, k, out_k, k_tok_stride, k_head_stride, hk, dt, bsz,
                     seq_len, hd, inv_freq, NULL, 0, 0, NULL, R, position, positions, position_ids, q_norm, k_norm,
                     nwt, eps, cb, mode, attn_factor, nthreads);
}

/* rope.cu:69-83 (inv_freq_table): the angle of frequency t is table[b * stride + pos * R/2 + t] */
int oracle_rope_table(const void* q, void* out_q, int64_t q_tok_stride, int64_t q_head_stride, int hq,
                      const void* k, void* out_k, int64_t k_tok_stride, int64_t k_head_stride, int hk,
                      int dt, int64_t bsz, int64_t seq_len, int hd,
                      const float* table, int64_t table_rows, int64_t table_bstride, int R,
                      int32_t position, const int32_t* positions, const int32_t* position_ids,
                      const void* q_norm, const void* k_norm, int nwt,
                      float eps, float cb, int mode, float attn_factor, int32_t* err, int nthreads)
{
    if (!table || table_rows <= 0 || table_bstride < 0) return -1;
    return rope_impl(q, out_q, q_tok_stride, q_head_stride, hq, k, out_k, k_tok_stride, k_head_stride, hk, dt, bsz,
                     seq_len, hd, NULL, table, table_rows, table_bstride, err, R, position, positions, position_ids,
                     q_norm, k_norm, nwt, eps, cb, mode, attn_factor, nthreads);
}

/* ------------------------------------------------------------------------------------------ */
/* Embedding gather: out[i] = table[ids[i]] (src/modules.rs:430-436: index_select, then an exact
 * to_kind(Float) upcast).  Out-of-range ids: zero row, *err_flag = 1. */
static inline int64_t load_id(const void* ids, int idt, int64_t i)
{
    return idt == OR_I64 ? ((const int64_t*)ids)[i] : (int64_t)((const int32_t*)ids)[i];
}

static size_t dsize(int dt) { return dt == OR_F32 ? 4 : 2; }

static int exact_conv(int from, int to) { return from == to || to == OR_F32; }

/* torch.argmax over each row (first maximal index, NaN maximal); kernels/generator/sampling_basic.cu:65-92 */
int oracle_argmax(const void* logits, int dt, int64_t rows, int64_t vocab, int64_t ldl, int max_logit, int64_t* ids,
                  int nthreads)
{
    if (!logits || !ids || rows < 0 || vocab <= 0 || ldl < vocab) return -1;
    if (!fdtype(dt)) return -2;
    int64_t n = (max_logit <= 0 || max_logit > vocab || oracle_mutation == ORM_ARGMAX_NO_MASK) ? vocab : max_logit;
    #pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int64_t i = 0; i < rows; ++i)
    {
        int64_t best = 0;
        float bv = ld(logits, dt, i * ldl + 0);
        for (int64_t j = 1; j < n; ++j)
        {
            const float v = ld(logits, dt, i * ldl + j);
            if (isnan(bv)) break;                                   /* the first NaN is final */
            const int better = isnan(v) || v > bv || (oracle_mutation == ORM_ARGMAX_LAST_TIE && v == bv);
            if (better) { bv = v; best = j; }
        }
        ids[i] = best;
    }
    return 0;
}

/* kernels/quant/hadamard.cu:88-170, hadamard_inner.cuh:96-200 */
int oracle_had_r_128(const void* x, int dt, int64_t ldx, void* out, int64_t ldo, int64_t rows, int64_t cols,
                     const uint16_t* pre, const uint16_t* post, float scale, int nthreads)
{
    if (!x || !out || rows < 0 || cols < 0 || cols % 128 || ldx < cols || ldo < cols || (pre && post)) return -1;
    if (dt != OR_F16 && dt != OR_F32) return -2;
    const float r = scale * 0.0883883461356163f;        /* fl32(1/sqrt(128)) */
    #pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int64_t i = 0; i < rows; ++i)
    {
        float v[128];
        for (int64_t b0 = 0; b0 < cols; b0 += 128)
        {
            for (int k = 0; k < 128; ++k)
            {
                float e = ld(x, dt, i * ldx + b0 + k);
                if (pre)
                {
                    const float p = oracle_f16_to_f32(pre[b0 + k]);
                    if (dt == OR_F16 && oracle_mutation != ORM_HAD_NO_PRE_ROUND)
                        e = oracle_f16_to_f32(oracle_f32_to_f16(e * p));    /* __hmul2: one half rounding */
                    else
                        e = e * p;
                }
                v[k] = e;
            }
            for (int h = 1; h < 128; h <<= 1)
                for (int k = 0; k < 128; ++k)
                    if (!(k & h))
                    {
                        const float a = v[k], c = v[k | h];
                        v[k] = a + c;
                        v[k | h] = (oracle_mutation == ORM_HAD_SIGN && h == 64) ? c - a : a - c;
                    }
            for (int k = 0; k < 128; ++k)
            {
                float e = v[k] * r;
                if (dt == OR_F16) e = oracle_f16_to_f32(oracle_f32_to_f16(e));
                if (post)
                {
                    const float p = oracle_f16_to_f32(post[b0 + k]);
                    e = dt == OR_F16 ? oracle_f16_to_f32(oracle_f32_to_f16(e * p)) : e * p;
                }
                st(out, dt, i * ldo + b0 + k, e);
            }
        }
    }
    return 0;
}

/* Philox4x32-10 (Salmon et al., SC 2011): ten rounds of two 32x32->64 multiplies with the published
 * multipliers and Weyl key increments. */
void oracle_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4])
{
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3], k0 = key[0], k1 = key[1];
    for (int round = 0; round < 10; ++round)
    {
        const uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0, n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        c1 = (uint32_t)p1;
        c3 = (uint32_t)p0;
        c0 = n0;
        c2 = n2;
        if (oracle_mutation != ORM_PHILOX_NO_BUMP) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

float oracle_log_f32(float x)
{
    uint32_t ix;
    memcpy(&ix, &x, 4);
    /* x = 2^e * m with m in [sqrt(1/2), sqrt(2)): 0x3f3504f3 is the bit pattern of sqrt(1/2) */
    const int32_t e = ((int32_t)(ix - 0x3f3504f3u)) >> 23;
    const uint32_t im = ix - ((uint32_t)e << 23);
    float m;
    memcpy(&m, &im, 4);
    const float f = m - 1.0f;                       /* exact */
    /* s = f / (2 + f) through 1/d: the linear minimax seed of 1/d on [2 - 0.2929, 2 + 0.4143]
     * (relative error 1.49e-2) and two Newton steps (5.0e-8); s only enters the correction term. */
    const float d = 2.0f + f;
    float y = fmaf(d, -0x1.e9813ap-3f, 0x1.f859fcp-1f);
    y = fmaf(y, fmaf(-d, y, 1.0f), y);
    y = fmaf(y, fmaf(-d, y, 1.0f), y);
    const float s = f * y;
    const float z = s * s;
    /* R = sum_{k=1..5} 2 s^2k / (2k + 1); coefficients are the floats nearest 2/3, 2/5, 2/7, 2/9, 2/11 */
    const float R = z * fmaf(z, fmaf(z, fmaf(z, fmaf(z, 0x1.745d18p-3f, 0x1.c71c72p-3f), 0x1.24924ap-2f),
                                      0x1.99999ap-2f), 0x1.555556p-1f);
    const float hfsq = 0.5f * f * f;
    const float ef = (float)e;
    const float lo = oracle_mutation == ORM_LOG_NO_LN2LO ? 0.0f : ef * 0x1.7f7d1cp-20f;
    /* ln2 = ln2_hi + ln2_lo; e * ln2_hi is exact: ln2_hi = 0x1.62e4p-1 (0.693145751953125) has 15
     * significant bits and |e| < 2^9, so the final fma rounds once, as a product and a difference would.
     * ln2_lo is the float nearest to ln2 - ln2_hi. */
    return fmaf(ef, 0x1.62e4p-1f, -((hfsq - fmaf(s, hfsq + R, lo)) - f));
}

static inline float gumbel_of_bits(uint32_t b)
{
    const float u = ((float)(b >> 9) + 0.5f) * 1.1920928955078125e-07f;    /* 2^-23 */
    return -oracle_log_f32(-oracle_log_f32(u));
}

void oracle_gumbel_of_bits(const uint32_t* bits, float* g, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) g[i] = gumbel_of_bits(bits[i]);
}

static inline float gumbel_at(uint32_t seed, int64_t r, int64_t c)
{
    if (oracle_mutation == ORM_GUMBEL_NO_ROW) r = 0;
    const uint32_t ctr[4] = { (uint32_t)(c >> 2), (uint32_t)r, (uint32_t)((uint64_t)r >> 32), 0 };
    const uint32_t key[2] = { seed, 0 };
    uint32_t out[4];
    oracle_philox4x32_10(ctr, key, out);
    return gumbel_of_bits(out[c & 3]);
}

int oracle_gumbel_noise(const void* x, int xt, int64_t ldx, void* out, int ot, int64_t ldo, int64_t rows,
                        int64_t cols, uint32_t seed, int nthreads)
{
    if (!x || !out || rows < 0 || cols < 0 || ldx < cols || ldo < cols) return -1;
    if (!fdtype(xt) || !fdtype(ot)) return -2;
    #pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < cols; ++c)
            st(out, ot, r * ldo + c, ld(x, xt, r * ldx + c) + gumbel_at(seed, r, c));
    return 0;
}

int oracle_gumbel_sample(const void* logits, int dt, int64_t rows, int64_t vocab, int64_t ldl, int max_logit,
                         uint32_t seed, int64_t* ids, int nthreads)
{
    if (!logits || !ids || rows < 0 || vocab <= 0 || ldl < vocab) return -1;
    if (!fdtype(dt)) return -2;
    const int64_t n = (max_logit <= 0 || max_logit > vocab) ? vocab : max_logit;
    #pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int64_t i = 0; i < rows; ++i)
    {
        int64_t best = 0;
        float bv = ld(logits, dt, i * ldl) + gumbel_at(seed, i, 0);
        for (int64_t j = 1; j < n && !isnan(bv); ++j)
        {
            const float v = ld(logits, dt, i * ldl + j) + gumbel_at(seed, i, j);
            if (isnan(v) || v > bv) { bv = v; best = j; }
        }
        ids[i] = best;
    }
    return 0;
}

/* kernels/norm.cu:482-581 (kernel), 591-668 (host rules) */
int oracle_gated_rms_norm(const void* x, int xt, int64_t ldx, const void* w, int wt, int w_groups,
                          void* y, int yt, int64_t ldy, const void* g, int gt, int64_t ldg,
                          int64_t rows, int64_t dim, float eps, float cb, int gate_first, int gate_act,
                          int nthreads)
{
    if (!x || !y || !g || dim <= 0 || rows < 0 || w_groups < 1) return -1;
    if (!fdtype(xt) || !fdtype(yt) || !fdtype(gt) || (w && !fdtype(wt))) return -2;
    if (gate_act != 0 && gate_act != 1) return -1;
    if (oracle_mutation == ORM_GATED_ORDER) gate_first = 0;
    const int act = gate_act ? OR_ACT_SIGMOID : OR_ACT_SILU;
    #pragma omp parallel num_threads(nthr(nthreads))
    {
        float* v = (float*)malloc((size_t)dim * sizeof(float));
        float* a = (float*)malloc((size_t)dim * sizeof(float));
        #pragma omp for schedule(static)
        for (int64_t i = 0; i < rows; ++i)
        {
            const int64_t wrow = oracle_mutation == ORM_GATED_WGROUP ? 0 : (i % w_groups) * dim;
            double s = 0.0;
            for (int64_t j = 0; j < dim; ++j)
            {
                a[j] = (float)act_d(act, (double)ld(g, gt, i * ldg + j));
                const float xv = ld(x, xt, i * ldx + j);
                v[j] = gate_first ? xv * a[j] : xv;
                s += (double)v[j] * (double)v[j];
            }
            const float rmf = 1.0f / sqrtf((float)s / (float)dim + eps);
            for (int64_t j = 0; j < dim; ++j)
            {
                float wv = 1.0f;
                if (w)
                {
                    wv = ld(w, wt, wrow + j);
                    if (cb != 0.0f) wv = wv + cb;
                }
                float o = w ? (v[j] * wv) * rmf : v[j] * rmf;
                if (!gate_first) o = o * a[j];
                st(y, yt, i * ldy + j, o);
            }
        }
        free(v);
        free(a);
    }
    return 0;
}

/* kernels/activation.cu:721-779 */
int oracle_deinterleave_qg(const void* qg, int64_t ldqg, void* q, int64_t ldq, void* g, int64_t ldg,
                           int64_t rows, int heads, int hd, int nthreads)
{
    if (!qg || !q || !g || rows < 0 || heads <= 0 || hd <= 0) return -1;
    void* dq = oracle_mutation == ORM_QG_SWAP ? g : q;
    void* dg = oracle_mutation == ORM_QG_SWAP ? q : g;
    #pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int64_t i = 0; i < rows; ++i)
        for (int h = 0; h < heads; ++h)
        {
            const char* src = (const char*)qg + (i * ldqg + (int64_t)h * 2 * hd) * 2;
            memcpy((char*)dq + (i * ldq + (int64_t)h * hd) * 2, src, (size_t)hd * 2);
            memcpy((char*)dg + (i * ldg + (int64_t)h * hd) * 2, src + (size_t)hd * 2, (size_t)hd * 2);
        }
    return 0;
}

/* kernels/generator/cache.cu:159-183 (index arithmetic), 186-243 (shape rules) */
int oracle_paged_kv_append(const void* k, int64_t k_tok_stride, int64_t k_head_stride,
                           const void* v, int64_t v_tok_stride, int64_t v_head_stride,
                           int hk, int dt, int64_t bsz, int64_t seq_len, int hd,
                           void* k_cache, void* v_cache, int page_size, int64_t num_pages,
                           const int32_t* block_table, int64_t max_blocks, const int32_t* cache_seqlens,
                           int32_t* err_flag, int nthreads)
{
    if (dt != OR_F16 && dt != OR_BF16) return -2;
    if (hk <= 0 || hd <= 0 || page_size <= 0 || num_pages <= 0 || max_blocks <= 0 || bsz < 0 || seq_len < 0) return -1;
    if (!block_table || !cache_seqlens || (k && !k_cache) || (v && !v_cache)) return -1;
    const size_t row = (size_t)hd * 2;
    int bad = 0;
    #pragma omp parallel for num_threads(nthr(nthreads)) reduction(|:bad) schedule(static)
    for (int64_t tok = 0; tok < bsz * seq_len; ++tok)
    {
        const int64_t b = tok / seq_len, s = tok % seq_len;
        int64_t pos = (int64_t)cache_seqlens[b] + s;
        if (oracle_mutation == ORM_PAGE_OFF) pos += 1;
        const int64_t lb = pos >= 0 ? pos / page_size : -1;
        const int64_t page = (lb >= 0 && lb < max_blocks) ? (int64_t)block_table[b * max_blocks + lb] : -1;
        if (page < 0 || page >= num_pages) { bad = 1; continue; }
        const int64_t dst_tok = page * page_size + pos % page_size;
        for (int h = 0; h < hk; ++h)
        {
            const int64_t dst = (dst_tok * hk + h) * hd;
            if (k) memcpy((char*)k_cache + dst * 2, (const char*)k + (tok * k_tok_stride + h * k_head_stride) * 2, row);
            if (v) memcpy((char*)v_cache + dst * 2, (const char*)v + (tok * v_tok_stride + h * v_head_stride) * 2, row);
        }
    }
    if (bad && err_flag) *err_flag = 1;
    return 0;
}

int oracle_embedding(const void* table, int tt, int64_t vocab, int64_t hidden, int64_t ldt,
                     const void* ids, int idt, int64_t n, void* out, int ot, int64_t ldo,
                     int32_t* err_flag, int nthreads)
{
    if (!table || !ids || !out || vocab <= 0 || hidden <= 0 || n < 0) return -1;
    if (!fdtype(tt) || !fdtype(ot) || (idt != OR_I32 && idt != OR_I64) || !exact_conv(tt, ot)) return -2;
    int bad = 0;
    #pragma omp parallel for num_threads(nthr(nthreads)) schedule(static) reduction(|:bad)
    for (int64_t i = 0; i < n; ++i)
    {
        int64_t id = load_id(ids, idt, i);
        if (oracle_mutation == ORM_EMBED_OFF) id += 1;
        if (id < 0 || id >= vocab)
        {
            bad = 1;
            for (int64_t j = 0; j < hidden; ++j) st(out, ot, i * ldo + j, 0.0f);
            continue;
        }
        if (ot == tt)   /* index_select is a bit copy (NaN payloads included) */
            memcpy((char*)out + i * ldo * dsize(ot), (const char*)table + id * ldt * dsize(tt), (size_t)hidden * dsize(tt));
        else
            for (int64_t j = 0; j < hidden; ++j) st(out, ot, i * ldo + j, ld(table, tt, id * ldt + j));
    }
    if (bad && err_flag) *err_flag = 1;
    return 0;
}

int oracle_embedding_rms_norm(const void* table, int tt, int64_t vocab, int64_t hidden, int64_t ldt,
                              const void* ids, int idt, int64_t n,
                              void* h, int ht, int64_t ldh,
                              const void* w, int wt, void* y, int yt, int64_t ldy,
                              float eps, float cb, float cs, int32_t* err_flag, int nthreads)
{
    if (!table || !ids || !y || vocab <= 0 || hidden <= 0 || n < 0) return -1;
    if (!fdtype(tt) || !fdtype(yt) || (w && !fdtype(wt)) || (idt != OR_I32 && idt != OR_I64)) return -2;
    if (h && (!fdtype(ht) || !exact_conv(tt, ht))) return -2;
    float* wf = weight_f32(w, wt, hidden, cb);
    int bad = 0;
    #pragma omp parallel num_threads(nthr(nthreads)) reduction(|:bad)
    {
        float* row = (float*)malloc((size_t)hidden * sizeof(float));
        #pragma omp for schedule(static)
        for (int64_t i = 0; i < n; ++i)
        {
            int64_t id = load_id(ids, idt, i);
            if (oracle_mutation == ORM_EMBED_OFF) id += 1;
            int ok = id >= 0 && id < vocab;
            if (!ok) bad = 1;
            for (int64_t j = 0; j < hidden; ++j) row[j] = ok ? ld(table, tt, id * ldt + j) : 0.0f;
            if (h && ht == tt && ok)
                memcpy((char*)h + i * ldh * dsize(ht), (const char*)table + id * ldt * dsize(tt), (size_t)hidden * dsize(tt));
            else if (h)
                for (int64_t j = 0; j < hidden; ++j) st(h, ht, i * ldh + j, row[j]);
            rms_row(row, wf, y, yt, i * ldy, hidden, eps, cs);
        }
        free(row);
    }
    free(wf);
    if (bad && err_flag) *err_flag = 1;
    return 0;
}
