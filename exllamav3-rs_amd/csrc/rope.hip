// Fused per-head RMSNorm + rotary embedding for gfx950: exl3r_rope (replaces exl3_shim_rope,
// reference csrc/exl3_shim.cpp:87-98 -> rope / rope_gr, kernels/rope.cu:279-467).
//
// Semantics follow rope_kernel (kernels/rope.cu:16-255):
//   position of token s of sequence b: position + s | positions[b] + s | position_ids[b*seq + s]
//   (rope.cu:55-67); head RMSNorm iff q_norm is given (rope.cu:250): sum of squares over the head
//   (carried in fp64), rmf = 1 / sqrt(sum / head_dim + eps) (IEEE fp32); f16 weights with f16 heads round twice in half precision,
//   out = h(h(w + cb) * h(v * rmf)) (rope.cu:222-229); other weights out = io((v * rmf) * (w + cb))
//   (rope.cu:212-221); the rotation reads the io-rounded normed head: angle = inv_freq[t] * (float)pos,
//   cos/sin * attn_factor (rope.cu:69-85), NeoX pairs (t, t + R/2), GPT-J pairs (2t, 2t+1), each
//   result rounded once (rope.cu:152-185); dims >= R pass through.
//   sin/cos are fp64 evaluations of the fp32 angle rounded once (positions reach 3e4 and beyond),
//   not the reference's __sinf/__cosf; the head sum is a full xor-butterfly sum in every lane (the reference's
//   shfl_down sum stored from all lanes, rope.cu:190-204, is only correct in lane 0).
//
// Layout: one workgroup per token (decode: several per token, splitting the heads).  A head of
// head_dim elements is held by LPH = head_dim / 8 lanes, 8 elements (16 bytes) per lane, so a wave
// holds 64 / LPH heads (4 heads of 128).  The head sum is a DPP butterfly inside the LPH-lane group;
// NeoX partners live R/16 lanes apart in the same group and are exchanged with ds_bpermute, GPT-J
// partners sit in the same lane.  sin/cos are computed once per (token, frequency) into LDS and
// shared by every head of the token.
#include "abi.hpp"
#include "common.cuh"

namespace exl3r {

struct RopeArgs
{
    const void* q;
    void* oq;
    const void* k;
    void* ok;
    int64_t q_ts, q_hs, k_ts, k_hs;   // token / head strides (elements)
    int hq, hk, hd, R;
    int64_t seq_len, tokens;
    const float* inv_freq;
    int32_t position;
    const int32_t* positions;
    const int32_t* position_ids;
    const void* qw;
    const void* kw;
    int wt;
    float eps, cb, attn;
    int tok_span;       // tokens spanned by one workgroup's item range (k_rope)
};

enum { NORM_NONE = 0, NORM_HALF = 1, NORM_F32 = 2 };

__device__ __forceinline__ int token_position(const RopeArgs& a, int tok)
{
    const int seq = (int)a.seq_len;
    const int b = tok / seq;
    const int s = tok - b * seq;
    if (a.positions) return a.positions[b] + s;
    if (a.position_ids) return a.position_ids[tok];
    return a.position + s;
}

// {cos, sin} * attn_factor of rotary frequency t at position pos: fp64 evaluation of the fp32
// angle, rounded once (correctly rounded fp32 values).
__device__ __forceinline__ float2 rope_cs(const RopeArgs& a, int t, int pos)
{
    const float ang = __fmul_rn(a.inv_freq[t], (float)pos);
    double sd, cd;
    sincos((double)ang, &sd, &cd);
    return make_float2((float)cd * a.attn, (float)sd * a.attn);
}

// sin/cos of every rotary frequency of one token into LDS (generic kernel).
__device__ __forceinline__ void fill_sincos(const RopeArgs& a, int pos, float2* cs)
{
    for (int t = threadIdx.x; t < a.R / 2; t += blockDim.x) cs[t] = rope_cs(a, t, pos);
}

// Work item = one (token, head) pair; a workgroup takes a contiguous range of slots * ITERS items,
// which spans at most a.tok_span tokens.  Every head chunk is loaded first; the sin/cos of the
// spanned tokens are evaluated into LDS while those loads are in flight.
template <class IO, int MODE, int LPH, int ITERS, int NORM>
__global__ __launch_bounds__(256) void k_rope(RopeArgs a)
{
    extern __shared__ float2 cs[];            // [tok_span][R / 2]
    const int tid = threadIdx.x;
    const int slot = tid / LPH;
    const int lane = tid % LPH;
    const int slots = blockDim.x / LPH;
    const int nheads = a.hq + a.hk;
    const int R2 = a.R / 2;
    const int64_t items = a.tokens * nheads;
    const int64_t per_wg = (int64_t)slots * ITERS;
    const bool lane_ok = lane * 8 < a.hd;
    const int e0 = lane * 8;                  // first head element held by this lane

    for (int64_t i0 = (int64_t)blockIdx.x * per_wg; i0 < items; i0 += (int64_t)gridDim.x * per_wg)
    {
        const int tok0 = (int)(i0 / nheads);
        const int hfirst = (int)(i0 - (int64_t)tok0 * nheads);

        typename IO::Vec v[ITERS];
        char* optr[ITERS];
        int trel[ITERS], head[ITERS];
        bool act[ITERS];
        #pragma unroll
        for (int it = 0; it < ITERS; ++it)
        {
            int rel = hfirst + it * slots + slot;
            int tr = 0;
            while (rel >= nheads) { rel -= nheads; ++tr; }
            trel[it] = tr;
            head[it] = rel;
            const int tok = tok0 + tr;
            act[it] = tok < a.tokens && lane_ok;
            optr[it] = nullptr;
            if (act[it])
            {
                const char* ip;
                if (rel < a.hq)
                {
                    const int64_t off = ((int64_t)tok * a.q_ts + (int64_t)rel * a.q_hs) * IO::bytes;
                    ip = (const char*)a.q + off;
                    optr[it] = (char*)a.oq + off;
                }
                else
                {
                    const int64_t off = ((int64_t)tok * a.k_ts + (int64_t)(rel - a.hq) * a.k_hs) * IO::bytes;
                    ip = (const char*)a.k + off;
                    optr[it] = (char*)a.ok + off;
                }
                v[it] = load8s<IO>(ip, e0);
            }
        }

        for (int i = tid; i < a.tok_span * R2; i += blockDim.x)
        {
            const int tr = i / R2;
            const int tok = tok0 + tr;
            if (tok < a.tokens) cs[i] = rope_cs(a, i - tr * R2, token_position(a, tok));
        }
        __syncthreads();

        #pragma unroll
        for (int it = 0; it < ITERS; ++it)
        {
            const float2* csr = cs + trel[it] * R2;
            float f[8];
            if (act[it]) unpack8<IO>(v[it], f);
            else
            {
                #pragma unroll
                for (int j = 0; j < 8; ++j) f[j] = 0.0f;
            }

            if constexpr (NORM != NORM_NONE)
            {
                // Sum of squares in fp64 (squares of 16-bit values are exact), one rounding to fp32:
                // the normed head is then bit-identical to a double-precision evaluation, so the
                // rotation that follows cannot amplify a last-bit difference through cancellation.
                double ss = 0.0;
                #pragma unroll
                for (int j = 0; j < 8; ++j) ss = fma((double)f[j], (double)f[j], ss);
                ss = group_sum64<LPH>(ss);
                const float rmf = rms_factor(ss, a.hd, a.eps);
                if (act[it])
                {
                    const void* w = head[it] < a.hq ? a.qw : a.kw;
                    if constexpr (NORM == NORM_HALF)
                    {
                        const TF16::Vec wv = load8<TF16>(w, e0);
                        const _Float16 cbh = to_f16(a.cb);
                        #pragma unroll
                        for (int j = 0; j < 8; ++j)
                        {
                            const uint32_t word = wv.a[j >> 1];
                            const _Float16 wh = __builtin_bit_cast(_Float16, (uint16_t)((j & 1) ? word >> 16 : word & 0xffffu)) + cbh;
                            const _Float16 nh = to_f16(f[j] * rmf);
                            f[j] = (float)(wh * nh);
                        }
                    }
                    else
                    {
                        float wf[8];
                        load8_dyn(w, a.wt, e0, wf);
                        #pragma unroll
                        for (int j = 0; j < 8; ++j) f[j] = round_to<IO>((f[j] * rmf) * (wf[j] + a.cb));
                    }
                }
            }

            // Rotation products rounded separately (no FMA contraction), as the reference semantics
            // state them: r1 = fl(fl(v1 c) - fl(v2 s)).
            if constexpr (MODE == EXL3R_ROPE_GPTJ)
            {
                #pragma clang fp contract(off)
                #pragma unroll
                for (int p = 0; p < 4; ++p)
                {
                    const int e = e0 + 2 * p;
                    if (e < a.R)
                    {
                        const float2 c = csr[e >> 1];
                        const float v1 = f[2 * p], v2 = f[2 * p + 1];
                        f[2 * p] = v1 * c.x - v2 * c.y;
                        f[2 * p + 1] = v2 * c.x + v1 * c.y;
                    }
                }
            }
            else
            {
                // Partner lane R/16 lanes away inside the head's lane group; values are exchanged as
                // packed io words (exact: they are io-rounded already).
                const int half = R2;
                const int dl = half >> 3;
                const bool rot = e0 < a.R;
                const bool lower = e0 < half;
                const int src_lane = rot ? (lower ? tid + dl : tid - dl) : tid;
                uint32_t other[4];
                const typename IO::Vec pk = pack8<IO>(f);
                #pragma unroll
                for (int i = 0; i < 4; ++i)
                    other[i] = (uint32_t)__builtin_amdgcn_ds_bpermute((src_lane & 63) << 2, (int)(uint32_t)pk.a[i]);
                if (rot)
                {
                    #pragma clang fp contract(off)
                    typename IO::Vec po;
                    #pragma unroll
                    for (int i = 0; i < 4; ++i) po.a[i] = other[i];
                    float g[8];
                    unpack8<IO>(po, g);
                    const int t0 = lower ? e0 : e0 - half;
                    #pragma unroll
                    for (int j = 0; j < 8; ++j)
                    {
                        const float2 c = csr[t0 + j];
                        f[j] = lower ? f[j] * c.x - g[j] * c.y : f[j] * c.x + g[j] * c.y;
                    }
                }
            }

            if (act[it]) store8<IO>(optr[it], (int64_t)e0, pack8<IO>(f));
        }
        __syncthreads();   // cs[] is refilled for the next range
    }
}

// Generic fallback (any even head_dim / rotary_dim, any alignment): one workgroup per token, heads
// walked serially through an LDS copy.
__global__ __launch_bounds__(256) void k_rope_generic(RopeArgs a, int dt, int mode, int norm)
{
    extern __shared__ float2 cs[];
    __shared__ double red[16];
    float* hv = (float*)(cs + a.R / 2);
    const int tid = threadIdx.x;
    const int half = a.R / 2;
    for (int64_t tok = blockIdx.x; tok < a.tokens; tok += gridDim.x)
    {
    fill_sincos(a, token_position(a, (int)tok), cs);
    __syncthreads();
    for (int head = 0; head < a.hq + a.hk; ++head)
    {
        const bool isq = head < a.hq;
        const void* ip = isq ? a.q : a.k;
        void* op = isq ? a.oq : a.ok;
        const int64_t off = isq ? tok * a.q_ts + (int64_t)head * a.q_hs : tok * a.k_ts + (int64_t)(head - a.hq) * a.k_hs;
        double ss = 0.0;
        for (int d = tid; d < a.hd; d += blockDim.x)
        {
            const float x = load1(ip, dt, off + d);
            hv[d] = x;
            ss = fma((double)x, (double)x, ss);
        }
        ss = block_sum64(ss, red);
        if (norm != NORM_NONE)
        {
            const float rmf = rms_factor(ss, a.hd, a.eps);
            const void* w = isq ? a.qw : a.kw;
            for (int d = tid; d < a.hd; d += blockDim.x)
            {
                if (norm == NORM_HALF)
                {
                    const _Float16 wh = ((const _Float16*)w)[d] + to_f16(a.cb);
                    hv[d] = (float)(wh * to_f16(hv[d] * rmf));
                }
                else
                    hv[d] = round1((hv[d] * rmf) * (load1(w, a.wt, d) + a.cb), dt);
            }
        }
        __syncthreads();
        for (int t = tid; t < half; t += blockDim.x)
        {
            #pragma clang fp contract(off)
            const int i1 = mode == EXL3R_ROPE_NEOX ? t : 2 * t;
            const int i2 = mode == EXL3R_ROPE_NEOX ? t + half : 2 * t + 1;
            const float v1 = hv[i1], v2 = hv[i2];
            hv[i1] = v1 * cs[t].x - v2 * cs[t].y;
            hv[i2] = v2 * cs[t].x + v1 * cs[t].y;
        }
        __syncthreads();
        for (int d = tid; d < a.hd; d += blockDim.x) store1(op, dt, off + d, hv[d]);
        __syncthreads();
    }
    }
}

template <class IO, int MODE, int LPH, int NORM>
static void launch_rope_lph(RopeArgs a, int iters, hipStream_t s)
{
    const int threads = 256;
    const int64_t per_wg = (int64_t)(threads / LPH) * iters;
    const int nheads = a.hq + a.hk;
    a.tok_span = (int)((nheads + per_wg - 2) / nheads) + 1;
    const int64_t items = a.tokens * nheads;
    int64_t blocks = (items + per_wg - 1) / per_wg;
    if (blocks > kMaxGridX) blocks = kMaxGridX;
    const size_t lds = (size_t)a.tok_span * (a.R / 2) * sizeof(float2);
    switch (iters)
    {
        case 1: k_rope<IO, MODE, LPH, 1, NORM><<<(unsigned)blocks, threads, lds, s>>>(a); break;
        case 2: k_rope<IO, MODE, LPH, 2, NORM><<<(unsigned)blocks, threads, lds, s>>>(a); break;
        default: k_rope<IO, MODE, LPH, 4, NORM><<<(unsigned)blocks, threads, lds, s>>>(a); break;
    }
}

// Items per lane: enough workgroups to fill 256 CUs several times over, then up to four heads per
// lane so each wave keeps 4 KiB of loads in flight.
template <class IO, int MODE, int NORM>
static void launch_rope_vec(const RopeArgs& a, int lph, hipStream_t s)
{
    const int64_t items = a.tokens * (a.hq + a.hk);
    const int64_t slots = 256 / lph;
    const Tuning& tu = tuning();
    int iters = 1;
    if (tu.rope_iters == 1 || tu.rope_iters == 2 || tu.rope_iters == 4) iters = tu.rope_iters;
    else if (items >= slots * 4 * 2048) iters = 4;
    else if (items >= slots * 2 * 2048) iters = 2;
    switch (lph)
    {
        case 1: launch_rope_lph<IO, MODE, 1, NORM>(a, iters, s); break;
        case 2: launch_rope_lph<IO, MODE, 2, NORM>(a, iters, s); break;
        case 4: launch_rope_lph<IO, MODE, 4, NORM>(a, iters, s); break;
        case 8: launch_rope_lph<IO, MODE, 8, NORM>(a, iters, s); break;
        case 16: launch_rope_lph<IO, MODE, 16, NORM>(a, iters, s); break;
        case 32: launch_rope_lph<IO, MODE, 32, NORM>(a, iters, s); break;
        default: launch_rope_lph<IO, MODE, 64, NORM>(a, iters, s); break;
    }
}

template <class IO>
static void launch_rope_io(const RopeArgs& a, int mode, int norm, int lph, hipStream_t s)
{
    auto go = [&](auto M) {
        constexpr int MODE = decltype(M)::value;
        if (norm == NORM_NONE) launch_rope_vec<IO, MODE, NORM_NONE>(a, lph, s);
        else if (norm == NORM_HALF) launch_rope_vec<IO, MODE, NORM_HALF>(a, lph, s);
        else launch_rope_vec<IO, MODE, NORM_F32>(a, lph, s);
    };
    if (mode == EXL3R_ROPE_GPTJ) go(std::integral_constant<int, EXL3R_ROPE_GPTJ>{});
    else go(std::integral_constant<int, EXL3R_ROPE_NEOX>{});
}

}  // namespace exl3r

using namespace exl3r;

extern "C" int exl3r_rope(const void* q, void* out_q, int64_t q_tok_stride, int64_t q_head_stride, int num_heads_q,
                          const void* k, void* out_k, int64_t k_tok_stride, int64_t k_head_stride, int num_heads_k,
                          int dtype, int64_t bsz, int64_t seq_len, int head_dim,
                          const float* inv_freq, int rotary_dim,
                          int32_t position, const int32_t* positions, const int32_t* position_ids,
                          const void* q_norm, const void* k_norm, int norm_dtype,
                          float norm_eps, float norm_constant_bias, int rope_mode, float attn_factor,
                          void* stream)
{
    const char* op = "exl3r_rope";
    if (!inv_freq) return set_error(EXL3R_EINVAL, "%s: inv_freq must be non-null", op);
    if (dtype != EXL3R_F16 && dtype != EXL3R_BF16)
        return set_error(EXL3R_EDTYPE, "%s: q/k dtype must be f16 or bf16, got %s", op, dtype_name(dtype));
    if (rope_mode != EXL3R_ROPE_GPTJ && rope_mode != EXL3R_ROPE_NEOX)
        return set_error(EXL3R_EINVAL, "%s: rope_mode must be GPTJ (1) or NEOX (2), got %d", op, rope_mode);
    if (bsz < 0 || seq_len < 0 || num_heads_q <= 0 || (k && num_heads_k <= 0))
        return set_error(EXL3R_EINVAL, "%s: invalid shape bsz=%lld seq_len=%lld heads=(%d,%d)", op, (long long)bsz,
                         (long long)seq_len, num_heads_q, num_heads_k);
    if (head_dim <= 0 || head_dim % 2 || head_dim > 4096)
        return set_error(EXL3R_EINVAL, "%s: head_dim %d must be even and in [2, 4096]", op, head_dim);
    if (rotary_dim < 2 || rotary_dim % 2 || rotary_dim > head_dim)
        return set_error(EXL3R_EINVAL, "%s: rotary_dim %d must be even and in [2, head_dim]", op, rotary_dim);
    if (q_head_stride < head_dim || q_tok_stride < (int64_t)num_heads_q * q_head_stride)
        return set_error(EXL3R_EINVAL, "%s: q strides (%lld, %lld) overlap heads", op, (long long)q_tok_stride, (long long)q_head_stride);
    if (k && ((bsz * seq_len > 0 && !out_k) || k_head_stride < head_dim || k_tok_stride < (int64_t)num_heads_k * k_head_stride))
        return set_error(EXL3R_EINVAL, "%s: k needs out_k and non-overlapping strides", op);
    if (positions && position_ids) return set_error(EXL3R_EINVAL, "%s: at most one of positions / position_ids", op);
    if (q_norm && k && !k_norm) return set_error(EXL3R_EINVAL, "%s: q_norm given without k_norm", op);
    if (!q_norm && k_norm) return set_error(EXL3R_EINVAL, "%s: k_norm given without q_norm", op);
    if (q_norm && !is_float_dtype(norm_dtype))
        return set_error(EXL3R_EDTYPE, "%s: unsupported norm weight dtype %s", op, dtype_name(norm_dtype));
    const int64_t tokens = bsz * seq_len;
    if (tokens == 0) return EXL3R_OK;
    if (!q || !out_q) return set_error(EXL3R_EINVAL, "%s: q and out_q must be non-null", op);
    if (tokens > 0x7fffffff) return set_error(EXL3R_EINVAL, "%s: too many tokens", op);

    RopeArgs a{};
    a.q = q; a.oq = out_q; a.k = k; a.ok = out_k;
    a.q_ts = q_tok_stride; a.q_hs = q_head_stride; a.k_ts = k_tok_stride; a.k_hs = k_head_stride;
    a.hq = num_heads_q; a.hk = k ? num_heads_k : 0; a.hd = head_dim; a.R = rotary_dim;
    a.seq_len = seq_len; a.tokens = tokens; a.inv_freq = inv_freq;
    a.position = position; a.positions = positions; a.position_ids = position_ids;
    a.qw = q_norm; a.kw = k_norm; a.wt = norm_dtype;
    a.eps = norm_eps; a.cb = norm_constant_bias; a.attn = attn_factor;
    const int norm = !q_norm ? NORM_NONE : (norm_dtype == EXL3R_F16 && dtype == EXL3R_F16) ? NORM_HALF : NORM_F32;
    hipStream_t s = (hipStream_t)stream;

    int lph = 1;
    while (lph * 8 < head_dim) lph *= 2;
    bool vec = head_dim % 8 == 0 && lph <= 64 && rotary_dim % (rope_mode == EXL3R_ROPE_NEOX ? 16 : 2) == 0;
    vec = vec && aligned16(q) && aligned16(out_q) && q_tok_stride % 8 == 0 && q_head_stride % 8 == 0;
    vec = vec && (!k || (aligned16(k) && aligned16(out_k) && k_tok_stride % 8 == 0 && k_head_stride % 8 == 0));
    vec = vec && (!q_norm || (aligned16(q_norm) && (!k_norm || aligned16(k_norm))));
    if (vec)
    {
        if (dtype == EXL3R_F16) launch_rope_io<TF16>(a, rope_mode, norm, lph, s);
        else launch_rope_io<TBF16>(a, rope_mode, norm, lph, s);
    }
    else
    {
        const size_t lds = (size_t)(rotary_dim / 2) * sizeof(float2) + (size_t)head_dim * sizeof(float);
        k_rope_generic<<<(unsigned)(tokens < kMaxGridX ? tokens : kMaxGridX), 256, lds, s>>>(a, dtype, rope_mode, norm);
    }
    return launch_status(op);
}
