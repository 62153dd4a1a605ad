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
//   sin/cos are double-precision evaluations of the fp32 angle rounded once (positions reach 3e4 and
//   beyond), not the reference's __sinf/__cosf; the head sum is a full xor-butterfly sum in every lane (the reference's
//   shfl_down sum stored from all lanes, rope.cu:190-204, is only correct in lane 0).
//
// Layout: a head of head_dim elements is held by LPH = head_dim / 8 lanes, 8 elements (16 bytes) per
// lane, so a wave holds 64 / LPH heads (4 heads of 128).  The head sum is a DPP butterfly inside the
// LPH-lane group; NeoX partners live R/16 lanes apart in the same group and are exchanged by DPP
// (a rotation by 8 lanes for R = 128) or ds_bpermute, GPT-J partners sit in the same lane.  Two
// kernels: k_rope_tok (prefill NeoX) gives each wave whole tokens -- the token's sin/cos evaluated
// once, one per lane, and its heads walked in software-pipelined batches; k_rope (decode, GPT-J)
// flattens (token, head) items over workgroups that share the sin/cos of the tokens they span
// through LDS.  exl3r_rope_cs_table evaluates the sin/cos of a forward pass once into a table
// that exl3r_rope_cs's kernels (the same two) copy rows of, instead of evaluating them per layer.
#include "abi.hpp"
#include "common.cuh"
#include "hadamard.cuh"

namespace exl3r {

struct RopeArgs
{
    const void* q;
    void* oq;
    const void* k;
    void* ok;
    int64_t q_ts, q_hs, k_ts, k_hs;   // token / head strides (elements)
    int64_t oq_ts, oq_hs;             // out_q's token / head strides (q's, except exl3r_rope_qg)
    int hq, hk, hd, R;
    int64_t seq_len, tokens;
    const float* inv_freq;
    // Angle table (exl3r_rope_table): angle of frequency t for token (b, s) at position pos is
    // table[b * table_bstride + pos * (R / 2) + t]; nullptr: angle = inv_freq[t] * pos.
    const float* table;
    int64_t table_rows, table_bstride;
    int32_t position;
    const int32_t* positions;
    const int32_t* position_ids;
    const void* qw;
    const void* kw;
    int wt;
    float eps, cb, attn;
    float inv_hd;       // 1 / head_dim when head_dim is a power of two, else 0
    int tok_span;       // tokens spanned by one workgroup's item range (k_rope)
    // Paged KV-cache append (exl3r_rope_paged_kv): v heads are copied and the roped k heads written
    // to caches [pages, 1 << page_log2, hk, hd]; kc == nullptr means no append.
    const void* v;
    int64_t v_ts, v_hs;
    int hv;             // v heads (hk with an append, else 0)
    void* kc;
    void* vc;
    int page_log2;
    int64_t pages, max_blocks;
    const int32_t* block_table;
    const int32_t* cache_seqlens;
    int32_t* err;
    // Output rotation of the q / k (and, with a paged append, v) projections (exl3r_rope_had,
    // exl3r_rope_paged_kv_had): each 128-element head is first replaced by had_r_128(head) times its
    // f16 post-scale (svh; nullptr: none).
    const void* q_post;
    const void* k_post;
    const void* v_post;
    // Precomputed rotary pairs (exl3r_rope_cs): {cos, sin} * attn_factor of frequency t for token
    // tok is cst[tok * (R / 2) + t]; nullptr: evaluated from inv_freq or the angle table.
    const float2* cst;
    // 8-lane kernel: the head norm's sum of squares in fp32 (1) instead of fp64 (sweep/test build only).
    int ss32;
    // 8-lane kernel: item / nslice as a multiply by ns_m and shifts by ns_l (udiv_magic), set at its launch.
    uint64_t ns_m;
    int ns_l;
};

// Unsigned division by an invariant d >= 1 as a multiply-high and two shifts (Granlund and Montgomery,
// "Division by invariant integers using multiplication", PLDI 1994, the round-up method): with
// l = ceil(log2 d) and m = floor(2^64 (2^l - d) / d) + 1 (below 2^64), n / d = (t + ((n - t) >> min(l, 1)))
// >> max(l - 1, 0) for t = mulhi(m, n), every n < 2^64.  For wave-uniform n it runs on the scalar unit and
// holds no vector register (the compiler's division keeps the divisor's float reciprocal in one).
static inline void udiv_magic_init(uint64_t d, uint64_t& m, int& l)
{
    l = 0;
    while (((uint64_t)1 << l) < d) ++l;
    m = (uint64_t)((((unsigned __int128)1 << 64) * (((uint64_t)1 << l) - d)) / d) + 1;
}
__device__ __forceinline__ uint64_t udiv_magic(uint64_t n, uint64_t m, int l)
{
    const uint64_t t = __umul64hi(m, n);
    return (t + ((n - t) >> (l < 1 ? l : 1))) >> (l > 1 ? l - 1 : 0);
}

// Where a kernel takes its rotary pairs: evaluated from inv_freq[t] * pos, evaluated from the angle
// table, or read from the precomputed {cos, sin} table.
enum { SRC_FREQ = 0, SRC_ANGLE = 1, SRC_CS = 2 };

// Head kinds of the item space [0, hq) q, [hq, hq + hk) k, [hq + hk, hq + hk + hv) v.
enum { KIND_Q = 0, KIND_K = 1, KIND_V = 2 };

__device__ __forceinline__ int head_kind(const RopeArgs& a, int h) { return h < a.hq ? KIND_Q : h < a.hq + a.hk ? KIND_K : KIND_V; }

// Element offset of token tok's row in the caches (cache_seqlens[b] + s through the block table,
// reference kernels/generator/cache.cu:173-179), or -1 after flagging a position outside the block
// table or a page outside the pool.
__device__ __forceinline__ int64_t cache_row(const RopeArgs& a, int64_t tok)
{
    const int64_t b = tok / a.seq_len;
    const int64_t pos = (int64_t)a.cache_seqlens[b] + (tok - b * a.seq_len);
    const int64_t lb = pos >> a.page_log2;
    const int64_t page = (pos >= 0 && lb < a.max_blocks) ? (int64_t)a.block_table[b * a.max_blocks + lb] : -1;
    if (page < 0 || page >= a.pages)
    {
        if (a.err) atomicOr(a.err, 1);
        return -1;
    }
    return ((page << a.page_log2) + (pos & (((int64_t)1 << a.page_log2) - 1))) * a.hk * a.hd;
}

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

// Wave-uniform forms of token_position and cache_row for kernels whose wave works on one token at a
// time: the index is moved to scalar registers and the int32 reads go through the scalar cache
// (constant address space), so their waits count only scalar loads and never the item data the wave
// has in flight (a vector read of the position or the block table would make its dependent use wait
// for every load issued before it).
__device__ __forceinline__ int64_t uniform64(int64_t v)
{
    const uint64_t u = (uint64_t)v;
    const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)u);
    const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
    return (int64_t)((hi << 32) | lo);
}
__device__ __forceinline__ int32_t scalar_i32(const int32_t* p, int64_t i)
{
    return ((const __attribute__((address_space(4))) int32_t*)p)[uniform64(i)];
}
// Sequence of token tok (< 2^31): a 32-bit division, none for a single sequence.
__device__ __forceinline__ int64_t token_seq_u(const RopeArgs& a, int64_t tok)
{
    return a.seq_len == a.tokens ? 0 : (int64_t)uniform64((uint32_t)tok / (uint32_t)a.seq_len);
}
__device__ __forceinline__ int token_position_u(const RopeArgs& a, int64_t tok)
{
    tok = uniform64(tok);
    const int64_t b = token_seq_u(a, tok);
    const int s = (int)(tok - b * a.seq_len);
    if (a.positions) return scalar_i32(a.positions, b) + s;
    if (a.position_ids) return scalar_i32(a.position_ids, tok);
    return a.position + s;
}
__device__ __forceinline__ int64_t cache_row_u(const RopeArgs& a, int64_t tok)
{
    tok = uniform64(tok);
    const int64_t b = token_seq_u(a, tok);
    const int64_t pos = (int64_t)scalar_i32(a.cache_seqlens, b) + (tok - b * a.seq_len);
    const int64_t lb = pos >> a.page_log2;
    const int64_t page = (pos >= 0 && lb < a.max_blocks) ? (int64_t)scalar_i32(a.block_table, b * a.max_blocks + lb) : -1;
    if (page < 0 || page >= a.pages)
    {
        if (a.err) atomicOr(a.err, 1);
        return -1;
    }
    return uniform64(((page << a.page_log2) + (pos & (((int64_t)1 << a.page_log2) - 1))) * a.hk * a.hd);
}

// sin and cos of an fp32 angle |a| < 2^52 in double precision (an int32 position times any
// inv_freq below 2^21), without the large-argument machinery of a general double sincos, which
// would cost ~30 VGPRs here.  Cody-Waite reduction a = k pi/2 + r with pi/2 split into three
// doubles: each FMA step is exact before its one rounding, so |r| <= pi/4 comes out with an
// absolute error near 2^-53 |r| for every k < 2^52.  Then the Taylor series of sin through r^15 and
// of cos through r^16 (truncation below 2^-54 on |r| <= pi/4).  Rounded to fp32 these agree with a
// libm double sin / cos of the same angle (checked on 4e7 angles: wide exponent range, inv_freq *
// position products, angles next to multiples of pi/2).  Larger angles give finite values with the
// wrong quadrant; no rotary table reaches them.
__device__ __forceinline__ void sincos_angle(float a, double& sd, double& cd)
{
    const double x = (double)a;
    const double k = rint(x * 0x1.45f306dc9c883p-1);            // 2 / pi
    double r = fma(-k, 0x1.921fb54442d18p+0, x);                // pi/2 = P1 + P2 + P3
    r = fma(-k, 0x1.1a62633145c07p-54, r);
    r = fma(-k, -0x1.f1976b7ed8fbcp-110, r);
    const double r2 = r * r;
    double ps = -0x1.ae7f3e733b81fp-41;                         // -1/15!
    ps = fma(ps, r2, 0x1.6124613a86d09p-33);                    //  1/13!
    ps = fma(ps, r2, -0x1.ae64567f544e4p-26);                   // -1/11!
    ps = fma(ps, r2, 0x1.71de3a556c734p-19);                    //  1/9!
    ps = fma(ps, r2, -0x1.a01a01a01a01ap-13);                   // -1/7!
    ps = fma(ps, r2, 0x1.1111111111111p-7);                     //  1/5!
    ps = fma(ps, r2, -0x1.5555555555555p-3);                    // -1/3!
    const double s = fma(r * r2, ps, r);
    double pc = 0x1.ae7f3e733b81fp-45;                          //  1/16!
    pc = fma(pc, r2, -0x1.93974a8c07c9dp-37);                   // -1/14!
    pc = fma(pc, r2, 0x1.1eed8eff8d898p-29);                    //  1/12!
    pc = fma(pc, r2, -0x1.27e4fb7789f5cp-22);                   // -1/10!
    pc = fma(pc, r2, 0x1.a01a01a01a01ap-16);                    //  1/8!
    pc = fma(pc, r2, -0x1.6c16c16c16c17p-10);                   // -1/6!
    pc = fma(pc, r2, 0x1.5555555555555p-5);                     //  1/4!
    pc = fma(pc, r2, -0.5);                                     // -1/2!
    const double c = fma(r2, pc, 1.0);
    const int q = (int)(k - 4.0 * floor(k * 0.25));             // k mod 4, exact for |k| < 2^53
    sd = q == 0 ? s : q == 1 ? c : q == 2 ? -s : -c;
    cd = q == 0 ? c : q == 1 ? -s : q == 2 ? -c : s;
}

// {cos, sin} * attn_factor of an fp32 angle.
__device__ __forceinline__ float2 rope_cs_of_angle(float ang, float attn)
{
    double sd, cd;
    sincos_angle(ang, sd, cd);
    return make_float2((float)cd * attn, (float)sd * attn);
}

// {cos, sin} * attn_factor of rotary frequency t for token tok at position pos: fp64 evaluation of
// the fp32 angle, rounded once (correctly rounded fp32 values).  SRC_ANGLE: the angle is read from
// the token's sequence row `pos` of the angle table; a position outside the table sets *err and
// rotates by 0.  SRC_CS: the pair is read from the precomputed table, which exl3r_rope_cs_table fills
// with this function's SRC_FREQ values.  (A compile-time choice: even a never-taken runtime branch
// here costs the prefill kernel ~5 us at C4 through its code generation.)
template <int SRC>
__device__ __forceinline__ float2 rope_cs(const RopeArgs& a, int t, int tok, int pos)
{
    if constexpr (SRC == SRC_CS) return a.cst[(int64_t)tok * (a.R >> 1) + t];
    float ang;
    if constexpr (SRC == SRC_ANGLE)
    {
        const int64_t b = tok / (int)a.seq_len;
        if (pos >= 0 && pos < a.table_rows) ang = a.table[b * a.table_bstride + (int64_t)pos * (a.R >> 1) + t];
        else
        {
            if (a.err) atomicOr(a.err, 1);
            ang = 0.0f;
        }
    }
    else ang = __fmul_rn(a.inv_freq[t], (float)pos);
    return rope_cs_of_angle(ang, a.attn);
}

// sin/cos of every rotary frequency of one token into LDS (generic kernel).
__device__ __forceinline__ void fill_sincos(const RopeArgs& a, int tok, int pos, float2* cs)
{
    for (int t = threadIdx.x; t < a.R / 2; t += blockDim.x)
        cs[t] = a.cst ? rope_cs<SRC_CS>(a, t, tok, pos) : a.table ? rope_cs<SRC_ANGLE>(a, t, tok, pos)
                                                                 : rope_cs<SRC_FREQ>(a, t, tok, pos);
}

// Norm weights of one lane's 8-element chunk with the constant bias folded in, loaded once per
// kernel: the packed half sums h(w + h(cb)) (NORM_HALF), or fp32 w + cb (NORM_F32).
template <int NORM> struct LaneW { };
template <> struct LaneW<NORM_HALF> { uint32_t a[4]; };
template <> struct LaneW<NORM_F32> { float f[8]; };

template <int NORM>
__device__ __forceinline__ LaneW<NORM> lane_weights(const RopeArgs& a, const void* w, int e0, bool ok)
{
    LaneW<NORM> r;
    if constexpr (NORM == NORM_HALF)
    {
        #pragma unroll
        for (int i = 0; i < 4; ++i) r.a[i] = 0;
        if (!ok || !w) return r;
        const TF16::Vec wv = load8<TF16>(w, e0);
        const _Float16 cbh = to_f16(a.cb);
        const f16x2 cb2 = { cbh, cbh };
        #pragma unroll
        for (int i = 0; i < 4; ++i) r.a[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, (uint32_t)wv.a[i]) + cb2);
    }
    else if constexpr (NORM == NORM_F32)
    {
        #pragma unroll
        for (int j = 0; j < 8; ++j) r.f[j] = 0.0f;
        if (!ok || !w) return r;
        load8_dyn(w, a.wt, e0, r.f);
        #pragma unroll
        for (int j = 0; j < 8; ++j) r.f[j] = r.f[j] + a.cb;
    }
    return r;
}

template <int NORM>
__device__ __forceinline__ LaneW<NORM> select_w(bool q, const LaneW<NORM>& wq, const LaneW<NORM>& wk)
{
    LaneW<NORM> r;
    if constexpr (NORM == NORM_HALF)
    {
        #pragma unroll
        for (int i = 0; i < 4; ++i) r.a[i] = q ? wq.a[i] : wk.a[i];
    }
    else if constexpr (NORM == NORM_F32)
    {
        #pragma unroll
        for (int j = 0; j < 8; ++j) r.f[j] = q ? wq.f[j] : wk.f[j];
    }
    return r;
}

// Head norm + rotation of the 8 elements e0 .. e0 + 7 one lane holds of a head spread over LPH
// lanes, in place on the lane's packed io chunk.  Must be called by the whole wave (the head sum
// and the NeoX exchange are cross-lane).
//   w:    the lane's weights (lane_weights) of this head's tensor;
//   c, s: cos / sin (times attn_factor) of the lane's frequencies: NeoX t0 .. t0 + 7 with
//         t0 = e0 mod R/2, GPT-J pairs (e0 + 2p, e0 + 2p + 1) in c[p], s[p] for p < 4;
//   l64:  lane index in the wave;
//   math: false leaves the chunk as loaded (v heads of a paged append; the cross-lane steps still run).
template <class IO, int MODE, int LPH, int NORM>
__device__ __forceinline__ void rope_head(const RopeArgs& a, typename IO::Vec& v, bool math, const LaneW<NORM>& w,
                                          const float (&c)[8], const float (&s)[8], int e0, int l64)
{
    if constexpr (NORM != NORM_NONE)
    {
        float f[8];
        unpack8<IO>(v, f);
        // Sum of squares in fp64 (squares of 16-bit values are exact), one rounding to fp32: the
        // normed head is then bit-identical to a double-precision evaluation, so the rotation that
        // follows cannot amplify a last-bit difference through cancellation.  sum / head_dim is a
        // multiply by the exact reciprocal when head_dim is a power of two (the same rounding).
        double ss = 0.0;
        #pragma unroll
        for (int j = 0; j < 8; ++j) ss = fma((double)f[j], (double)f[j], ss);
        ss = group_sum64<LPH>(ss);
        const float mean = a.inv_hd != 0.0f ? (float)ss * a.inv_hd : (float)ss / (float)a.hd;
        const float rmf = 1.0f / sqrtf(mean + a.eps);
        if (!math) {}
        else if constexpr (NORM == NORM_HALF)
        {
            // Two half roundings: h(w + h(cb)) * h(v * rmf), multiplied as packed halves.
            #pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                const f16x2 n2 = { to_f16(f[2 * i] * rmf), to_f16(f[2 * i + 1] * rmf) };
                v.a[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, (uint32_t)w.a[i]) * n2);
            }
        }
        else
        {
            #pragma unroll
            for (int j = 0; j < 8; ++j) f[j] = (f[j] * rmf) * w.f[j];
            v = pack8<IO>(f);
        }
    }

    // Rotation products rounded separately (no FMA contraction), as the reference semantics state
    // them: r1 = fl(fl(v1 c) - fl(v2 s)).
    if constexpr (MODE == EXL3R_ROPE_GPTJ)
    {
        if (math && e0 < a.R)
        {
            #pragma clang fp contract(off)
            float f[8];
            unpack8<IO>(v, f);
            #pragma unroll
            for (int p = 0; p < 4; ++p)
            {
                if (e0 + 2 * p < a.R)
                {
                    const float v1 = f[2 * p], v2 = f[2 * p + 1];
                    f[2 * p] = v1 * c[p] - v2 * s[p];
                    f[2 * p + 1] = v2 * c[p] + v1 * s[p];
                }
            }
            v = pack8<IO>(f);
        }
    }
    else
    {
        // The partner lane is dl = R/16 lanes away inside the head's lane group; the packed io words
        // are exchanged as they are.  R = 128 at 16 lanes per head is a rotation by 8 inside a DPP row.
        const int R2 = a.R >> 1;
        const int dl = R2 >> 3;
        const bool rot = e0 < a.R;
        const bool lower = e0 < R2;
        typename IO::Vec po;
        if (LPH == 16 && dl == 8)
        {
            #pragma unroll
            for (int i = 0; i < 4; ++i)
                po.a[i] = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v.a[i], DPP_ROW_ROR8, 0xf, 0xf, false);
        }
        else
        {
            const int src = rot ? (lower ? l64 + dl : l64 - dl) : l64;
            #pragma unroll
            for (int i = 0; i < 4; ++i)
                po.a[i] = (uint32_t)__builtin_amdgcn_ds_bpermute(src << 2, (int)(uint32_t)v.a[i]);
        }
        if (math && rot)
        {
            #pragma clang fp contract(off)
            float f[8], g[8];
            unpack8<IO>(v, f);
            unpack8<IO>(po, g);
            #pragma unroll
            for (int j = 0; j < 8; ++j) f[j] = f[j] * c[j] + g[j] * s[j];   // lower half: s holds -sin
            v = pack8<IO>(f);
        }
    }
}

// cos / sin of the lane's frequencies (rope_head's c, s) out of a row of R/2 {cos, sin} pairs.  NeoX
// lanes of the lower half take -sin, so every rotated lane computes v c + partner s: fl(v c) +
// fl(partner (-sin)) is fl(v c) - fl(partner sin) bit for bit (negation is exact and x - y is
// x + (-y)).
template <int MODE>
__device__ __forceinline__ void lane_sincos(const float2* row, int e0, int R, float (&c)[8], float (&s)[8])
{
    const int t0 = MODE == EXL3R_ROPE_GPTJ ? (e0 >> 1) : (e0 < (R >> 1) ? e0 : e0 - (R >> 1));
    #pragma unroll
    for (int j = 0; j < 8; ++j)
    {
        c[j] = s[j] = 0.0f;
        if (MODE == EXL3R_ROPE_NEOX ? e0 < R : (j < 4 && e0 + 2 * j < R))
        {
            const float2 x = row[t0 + j];
            c[j] = x.x;
            s[j] = MODE == EXL3R_ROPE_NEOX && e0 < (R >> 1) ? -x.y : x.y;
        }
    }
}

// Decode / small launches.  Work item = one (token, head) pair; a workgroup takes a contiguous range
// of slots * ITERS items, which spans at most a.tok_span tokens.  Every head chunk is loaded first;
// the sin/cos of the spanned tokens are evaluated into LDS while those loads are in flight.
template <class IO, int MODE, int LPH, int ITERS, int NORM, bool APPEND, int SRC>
__global__ __launch_bounds__(256) void k_rope(RopeArgs a)
{
    extern __shared__ float2 cs[];            // [tok_span][R / 2]
    const int tid = threadIdx.x;
    const int slot = tid / LPH;
    const int lane = tid % LPH;
    const int slots = blockDim.x / LPH;
    const int nheads = a.hq + a.hk + (APPEND ? a.hv : 0);
    const int R2 = a.R / 2;
    const int64_t items = a.tokens * nheads;
    const int64_t per_wg = (int64_t)slots * ITERS;
    const bool lane_ok = lane * 8 < a.hd;
    const int e0 = lane * 8;                  // first head element held by this lane
    const LaneW<NORM> wq = lane_weights<NORM>(a, a.qw, e0, lane_ok);
    const LaneW<NORM> wk = lane_weights<NORM>(a, a.kw, e0, lane_ok);

    for (int64_t i0 = (int64_t)blockIdx.x * per_wg; i0 < items; i0 += (int64_t)gridDim.x * per_wg)
    {
        const int tok0 = (int)(i0 / nheads);
        const int hfirst = (int)(i0 - (int64_t)tok0 * nheads);

        typename IO::Vec v[ITERS];
        char* optr[ITERS];      // io output (nullptr: none)
        char* cptr[ITERS];      // cache output (nullptr: none)
        int trel[ITERS], kind[ITERS];
        bool act[ITERS];
        #pragma unroll
        for (int it = 0; it < ITERS; ++it)
        {
            int rel = hfirst + it * slots + slot;
            int tr = 0;
            while (rel >= nheads) { rel -= nheads; ++tr; }
            trel[it] = tr;
            kind[it] = APPEND ? head_kind(a, rel) : rel < a.hq ? KIND_Q : KIND_K;
            const int tok = tok0 + tr;
            act[it] = tok < a.tokens && lane_ok;
            optr[it] = cptr[it] = nullptr;
            if (act[it])
            {
                const char* ip;
                if (kind[it] == KIND_Q)
                {
                    ip = (const char*)a.q + ((int64_t)tok * a.q_ts + (int64_t)rel * a.q_hs) * IO::bytes;
                    optr[it] = (char*)a.oq + ((int64_t)tok * a.oq_ts + (int64_t)rel * a.oq_hs) * IO::bytes;
                }
                else if constexpr (!APPEND)
                {
                    const int64_t off = ((int64_t)tok * a.k_ts + (int64_t)(rel - a.hq) * a.k_hs) * IO::bytes;
                    ip = (const char*)a.k + off;
                    optr[it] = (char*)a.ok + off;
                }
                else
                {
                    const int hkv = rel - a.hq - (kind[it] == KIND_V ? a.hk : 0);
                    if (kind[it] == KIND_K)
                    {
                        const int64_t off = ((int64_t)tok * a.k_ts + (int64_t)hkv * a.k_hs) * IO::bytes;
                        ip = (const char*)a.k + off;
                        if (a.ok) optr[it] = (char*)a.ok + off;
                    }
                    else
                        ip = (const char*)a.v + ((int64_t)tok * a.v_ts + (int64_t)hkv * a.v_hs) * IO::bytes;
                    if (APPEND)
                    {
                        const int64_t row = cache_row(a, tok);
                        if (row >= 0)
                            cptr[it] = (char*)(kind[it] == KIND_K ? a.kc : a.vc) + (row + (int64_t)hkv * a.hd) * IO::bytes;
                    }
                }
                v[it] = load8s<IO>(ip, e0);
            }
        }

        for (int i = tid; i < a.tok_span * R2; i += blockDim.x)
        {
            const int tr = i / R2;
            const int tok = tok0 + tr;
            if (tok < a.tokens) cs[i] = rope_cs<SRC>(a, i - tr * R2, tok, token_position(a, tok));
        }
        __syncthreads();

        #pragma unroll
        for (int it = 0; it < ITERS; ++it)
        {
            float c[8], s[8];
            if (!act[it])
            {
                #pragma unroll
                for (int i = 0; i < 4; ++i) v[it].a[i] = 0;
            }
            lane_sincos<MODE>(cs + trel[it] * R2, e0, a.R, c, s);
            rope_head<IO, MODE, LPH, NORM>(a, v[it], kind[it] != KIND_V, select_w<NORM>(kind[it] == KIND_Q, wq, wk), c, s,
                                           e0, tid & 63);
            if (act[it] && (!APPEND || optr[it])) store8<IO>(optr[it], (int64_t)e0, v[it]);
            if (APPEND && act[it] && cptr[it]) store8<IO>(cptr[it], (int64_t)e0, v[it]);
        }
        __syncthreads();   // cs[] is refilled for the next range
    }
}

// Orders one wave's LDS writes before its following LDS reads (and the reads before later writes)
// without a workgroup barrier.
__device__ __forceinline__ void wave_lds_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Prefill launches: one wave per token at a time.  The wave evaluates a token's R/2 {cos, sin}
// pairs once, one per lane, into its LDS row; each lane keeps the pairs its elements need in
// registers, and the wave walks the token's heads in batches of HPL passes (64/LPH heads per pass).
// The loads of the next batch are issued before the current batch is computed, and a new token's
// sin/cos are evaluated while its first batch is in flight, so every wave keeps loads in flight
// while it computes.  The four waves of a workgroup take different tokens and never wait for each
// other.
template <class IO, int HPL>
struct RopeBatch
{
    typename IO::Vec v[HPL];
    int32_t off[HPL];            // element offset of the lane's chunk inside its token's q, k or v row
    int32_t hidx[HPL];           // head index inside k or v (the cache row offset of an append)
    bool isq[HPL], isv[HPL];
    bool act[HPL];
    int64_t tok;
    int64_t crow;                // the token's cache row (cache_row), -1: no append
    int b;
};

template <class IO, int MODE, int LPH, int HPL, int NORM, bool APPEND, bool HADR = false, int SRC = SRC_FREQ,
          bool QOUT = false>
__global__ __launch_bounds__(256) void k_rope_tok(RopeArgs a)
{
    extern __shared__ float2 cs[];            // [4 waves][R / 2]
    constexpr int HPP = 64 / LPH;             // heads per pass
    const int l64 = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int sub = l64 / LPH;
    const int e0 = (l64 % LPH) * 8;
    const bool lane_ok = e0 < a.hd;
    const int R2 = a.R >> 1;
    const int nheads = a.hq + a.hk + (APPEND ? a.hv : 0);
    const int nb = ((nheads + HPP - 1) / HPP + HPL - 1) / HPL;    // batches per token
    const int64_t nwaves = (int64_t)gridDim.x * 4;
    float2* row = cs + wave * R2;
    const LaneW<NORM> wq = lane_weights<NORM>(a, a.qw, e0, lane_ok);
    const LaneW<NORM> wk = lane_weights<NORM>(a, a.kw, e0, lane_ok);
    // Per-lane choices between argument fields select values, not addresses: a selected field
    // address is read with a vector load from the argument segment on every use.
    const int64_t q_hs = a.q_hs, k_hs = a.k_hs, v_hs = APPEND ? a.v_hs : 0, oq_hs = a.oq_hs;
    auto head_stride = [&](int kind) { return kind == KIND_Q ? q_hs : kind == KIND_K ? k_hs : v_hs; };

    auto issue = [&](RopeBatch<IO, HPL>& t) {
        const char* qb = (const char*)a.q + t.tok * a.q_ts * IO::bytes;
        const char* kb = (const char*)a.k + t.tok * a.k_ts * IO::bytes;
        const char* vb = (const char*)a.v + t.tok * a.v_ts * IO::bytes;
        #pragma unroll
        for (int i = 0; i < HPL; ++i)
        {
            const int h = (t.b * HPL + i) * HPP + sub;
            t.act[i] = lane_ok && h < nheads;
            t.isq[i] = h < a.hq;
            t.isv[i] = APPEND && h >= a.hq + a.hk;
            const int kd = t.isq[i] ? KIND_Q : t.isv[i] ? KIND_V : KIND_K;
            t.hidx[i] = h - (kd == KIND_Q ? 0 : kd == KIND_K ? a.hq : a.hq + a.hk);
            t.off[i] = (int32_t)((int64_t)t.hidx[i] * head_stride(kd)) + e0;
            if (t.act[i]) t.v[i] = load8s<IO>(kd == KIND_Q ? qb : kd == KIND_K ? kb : vb, t.off[i]);
        }
    };
    float c[8], s[8];
    auto fill = [&](int64_t tok) {
        const int pos = token_position(a, (int)tok);
        wave_lds_sync();
        for (int t = l64; t < R2; t += 64) row[t] = rope_cs<SRC>(a, t, (int)tok, pos);
        wave_lds_sync();
        lane_sincos<MODE>(row, e0, a.R, c, s);
    };
    auto compute = [&](RopeBatch<IO, HPL>& t, const float (&c)[8], const float (&s)[8]) {
        char* qo = (char*)a.oq + t.tok * (QOUT ? a.oq_ts : a.q_ts) * IO::bytes;
        char* ko = (char*)a.ok + t.tok * a.k_ts * IO::bytes;
        #pragma unroll
        for (int i = 0; i < HPL; ++i)
        {
            if (!t.act[i])
            {
                #pragma unroll
                for (int j = 0; j < 4; ++j) t.v[i].a[j] = 0;
            }
            const int kd = t.isq[i] ? KIND_Q : t.isv[i] ? KIND_V : KIND_K;
            if constexpr (HADR)
            {
                // A head is one rotation block: head_dim 128, 16 lanes, all active or all not (a
                // padding head past the last one has no post-scale entries and is left alone).
                static_assert(IO::code == DT_F16 && LPH == 16, "output rotation: f16 heads of 128");
                const void* post = kd == KIND_Q ? a.q_post : kd == KIND_K ? a.k_post : a.v_post;
                if (t.act[i]) output_rotation8(t.v[i], post, (int64_t)t.hidx[i] * 128 + e0);
            }
            rope_head<IO, MODE, LPH, NORM>(a, t.v[i], kd != KIND_V, select_w<NORM>(kd == KIND_Q, wq, wk), c, s, e0, l64);
            if (!t.act[i]) continue;
            // QOUT: out_q has its own layout (exl3r_rope_qg).  A compile-time choice: the separate
            // offset costs the plain prefill kernel 7 us at C4 (45.6 vs 38.5 us).
            const int32_t qoff = QOUT ? (int32_t)((int64_t)t.hidx[i] * oq_hs) + e0 : t.off[i];
            if (!APPEND)
            {
                if (kd == KIND_Q) store8<IO>(qo, qoff, t.v[i]);
                else store8<IO>(ko, t.off[i], t.v[i]);
                continue;
            }
            if (kd == KIND_Q) store8<IO>(qo, qoff, t.v[i]);
            else
            {
                if (kd == KIND_K && a.ok) store8<IO>(ko, t.off[i], t.v[i]);
                if (APPEND && t.crow >= 0)
                    store8<IO>(kd == KIND_K ? a.kc : a.vc, t.crow + (int64_t)t.hidx[i] * a.hd + e0, t.v[i]);
            }
        }
    };

    RopeBatch<IO, HPL> A, B;
    A.tok = (int64_t)blockIdx.x * 4 + wave;
    A.b = 0;
    if (A.tok >= a.tokens) return;
    A.crow = APPEND ? cache_row(a, A.tok) : -1;
    issue(A);
    fill(A.tok);

    // One pipeline step: start `nxt` (the batch after `cur`), then finish `cur`.  Returns false
    // when `cur` was the wave's last batch.
    auto step = [&](RopeBatch<IO, HPL>& cur, RopeBatch<IO, HPL>& nxt) -> bool {
        nxt.tok = cur.tok;
        nxt.b = cur.b + 1;
        if (nxt.b == nb)
        {
            nxt.b = 0;
            nxt.tok += nwaves;
        }
        const bool more = nxt.tok < a.tokens;
        if (APPEND && more) nxt.crow = nxt.b == 0 ? cache_row(a, nxt.tok) : cur.crow;
        if (more) issue(nxt);
        compute(cur, c, s);
        if (more && nxt.b == 0) fill(nxt.tok);
        return more;
    };
    while (step(A, B) && step(B, A)) {}
}

// head_dim 128 at prefill sizes, NeoX with rotary_dim 128 (Qwen3, Llama) or GPT-J with any rotary_dim:
// 8 lanes per head, lane j of a head's group holding elements [8j, 8j + 8) and [64 + 8j, 64 + 8j + 8),
// so every rotary pair sits in one lane -- NeoX (t, t + 64) across the two chunks, GPT-J (2t, 2t + 1)
// inside a chunk -- with no partner exchange; the head sum is a 3-step DPP butterfly, and each 16-byte
// load or store instruction covers whole 128-byte lines of 8 heads.  An item is one pass
// of 8 heads of one token (items in token order, a token's q passes then its k pass).  Each wave
// walks runs of `run` consecutive items, run r of wave g being items [(g + r W) run, (g + r W + 1) run)
// (W waves in the grid), so the waves in flight sweep the rows in order; the next item's loads (and
// its {cos, sin} table row) are issued before the current item is computed.  Evaluated rotary pairs:
// one sin / cos per lane into the wave's LDS row, once per token within a run.
template <class IO, int NORM, int SRC, int P>
struct NxItem
{
    typename IO::Vec lo[P], hi[P];
    float4 cs[4];                // SRC_CS: the lane's 8 {cos, sin} pairs as loaded
    int64_t tok;
    int64_t crow;                // APPEND: the token's cache row (cache_row), -1: none or not needed
    int slice;
    int pos;                     // SRC_FREQ: the token's position
};

// One of three values by a per-lane choice (q / k / v heads), as mask arithmetic: hipcc turns a chain
// of selects between three values into a lookup table in scratch memory indexed per lane (~600 bytes
// per lane and twice the kernel time in the paged instances).
__device__ __forceinline__ uint64_t pick_qkv_bits(bool isq, bool isv, uint64_t q, uint64_t k, uint64_t v)
{
    const uint64_t mq = (uint64_t)0 - (uint64_t)isq, mv = (uint64_t)0 - (uint64_t)(!isq && isv);
    const uint64_t mk = ~(mq | mv);
    return (q & mq) | (k & mk) | (v & mv);
}
template <class T>
__device__ __forceinline__ T* pick_qkv(bool isq, bool isv, T* q, T* k, T* v)
{
    return (T*)pick_qkv_bits(isq, isv, (uint64_t)q, (uint64_t)k, (uint64_t)v);
}
__device__ __forceinline__ int64_t pick_qkv(bool isq, bool isv, int64_t q, int64_t k, int64_t v)
{
    return (int64_t)pick_qkv_bits(isq, isv, (uint64_t)q, (uint64_t)k, (uint64_t)v);
}

// The EXL3 linear's output rotation had_r_128(head) of one f16 head of 128 on the 8-lane layout (lane
// l8 of the head's group holds elements [8 l8, 8 l8 + 8) in lo and [64 + 8 l8, 64 + 8 l8 + 8) in hi):
// index bits 0-2 in-lane in both chunks, bits 3-5 lane exchanges at xor 1, 2, 4 inside the group, bit
// 6 the lo / hi pair -- the reference's order of stages (bits 0..6) and pairs (a, b) -> (a + b, a - b)
// in fp32, then the scale 1/sqrt(128) and one rounding to f16 (the post-scale product follows).
__device__ __forceinline__ void rotate_head_nx(TF16::Vec& lo, TF16::Vec& hi, int l8)
{
    #pragma clang fp contract(off)
    float fl[8], fh[8];
    unpack8_stage1(lo, fl);     // index bit 0 from the packed pairs
    unpack8_stage1(hi, fh);
    #pragma unroll
    for (int h = 2; h < 8; h <<= 1)
    {
        #pragma unroll
        for (int j = 0; j < 8; ++j)
        {
            if (j & h) continue;
            float a = fl[j], b = fl[j | h];
            fl[j] = a + b;
            fl[j | h] = a - b;
            a = fh[j];
            b = fh[j | h];
            fh[j] = a + b;
            fh[j | h] = a - b;
        }
    }
    lane_stage<1>(fl, l8);
    lane_stage<1>(fh, l8);
    lane_stage<2>(fl, l8);
    lane_stage<2>(fh, l8);
    lane_stage<4>(fl, l8);
    lane_stage<4>(fh, l8);
    #pragma unroll
    for (int j = 0; j < 8; ++j)
    {
        const float a = fl[j], b = fh[j];
        fl[j] = opaque((a + b) * 0.0883883461356163f);
        fh[j] = opaque((a - b) * 0.0883883461356163f);
    }
    lo = pack8<TF16>(fl);
    hi = pack8<TF16>(fh);
}

// APPEND: v heads follow the k heads in the item space; k and v rows are written to the paged caches
// (exl3r_rope_paged_kv).  HADR: every head is first replaced by its projection's output rotation
// (exl3r_rope_had, exl3r_rope_paged_kv_had), as the reference's butterfly (HADR_EXACT,
// rotate_head_nx) or on the matrix cores (HADR_MFMA).  Both take one pass per item.
// The rotating instances evaluating sin / cos, and the matrix-core ones reading the table, land just above
// the five-wave budget (97-100 VGPRs of 96); they are held to five waves per SIMD.
enum { HADR_NONE = 0, HADR_EXACT = 1, HADR_MFMA = 2 };
template <bool APPEND, int HADR, int SRC>
constexpr int kNxMinWaves = HADR && (SRC == SRC_FREQ || HADR == HADR_MFMA) ? 5 : 1;

// Lane layouts of a pass (8 heads of 128, 16 elements per lane: the chunks [e0, e0 + 8) and
// [e0 + 64, e0 + 72) of head grp, the NeoX pairs of the full rotary width side by side):
//  - the 8-lane layout: head grp = lane bits 3-5, e0 = 8 * (lane bits 0-2);
//  - the matrix-core layout (HADR_MFMA): head grp = lane bits 2, 3, 5, e0 = 8 * (lane bits 0, 1, 4).
//    The items are loaded as two 4-head spans in had128_mfma's placement (slot s: head 4 s + lane bits
//    2-3, chunk lane bits 0, 1, 4, 5 = index bits 3-6), transformed there, and moved to this layout by
//    one v_permlane32_swap per word pair: the swap exchanges lane bit 5 (index bit 6) with the slot
//    (head bit 2).  A head's 8 lanes are then lanes {0, 1, 4} of its group, so the head norm sums over
//    lanes xor 1, 2 and 16.
template <int HADR>
__device__ __forceinline__ int nx_head_of_lane(int l64)
{
    return HADR == HADR_MFMA ? ((l64 >> 2) & 3) | ((l64 >> 3) & 4) : l64 >> 3;
}
template <int HADR>
__device__ __forceinline__ int nx_e0_of_lane(int l64)
{
    return HADR == HADR_MFMA ? 8 * ((l64 & 3) | ((l64 >> 2) & 4)) : (l64 & 7) * 8;
}

// Sum over the 8 lanes of a head of a pass (every lane of the head gets the same bits).
template <int HADR>
__device__ __forceinline__ float nx_head_sum(float v)
{
    if constexpr (HADR == HADR_MFMA)
    {
        v += dpp<DPP_QUAD_XOR1>(v);
        v += dpp<DPP_QUAD_XOR2>(v);
        return sum_xor16(v);
    }
    else
        return group_sum<8>(v);
}
template <int HADR>
__device__ __forceinline__ double nx_head_sum(double v)
{
    if constexpr (HADR == HADR_MFMA)
    {
        v += dpp64<DPP_QUAD_XOR1>(v);
        v += dpp64<DPP_QUAD_XOR2>(v);
        return sum_xor16(v);
    }
    else
        return group_sum64<8>(v);
}

template <class IO, int MODE, int NORM, int SRC, bool QOUT, int P, bool APPEND = false, int HADR = HADR_NONE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(kNxMinWaves<APPEND, HADR, SRC>)))
void k_rope_nx(RopeArgs a, int nslice, int run)
{
    static_assert(!(APPEND || HADR) || (P == 1 && !QOUT), "paged / rotating items are single passes");
    static_assert(!HADR || IO::code == DT_F16, "output rotation: f16 heads");
    extern __shared__ float2 cs[];            // [4 waves][64] (SRC_FREQ)
    // Norm weights with the constant bias folded in, q then k: h(w + h(cb)) (NORM_HALF) or w + cb (NORM_F32).
    __shared__ __align__(16) float wsh[256];
    static_assert(SRC == SRC_FREQ || SRC == SRC_CS, "angle tables take the flattened kernel");
    const int l64 = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t W = (int64_t)gridDim.x * 4;
    const int64_t items = a.tokens * nslice;
    const int grp = nx_head_of_lane<HADR>(l64);   // head of a pass held by this lane
    const int e0 = nx_e0_of_lane<HADR>(l64);      // the lane's chunks: [e0, e0 + 8) and [e0 + 64, e0 + 72)
    constexpr bool MF = HADR == HADR_MFMA;
    // had128_mfma's placement: the lane's chunk of each span (index bits 3-6 = lane bits 0, 1, 4, 5) and
    // its head inside the span (lane bits 2-3).
    const int mf_e = 8 * ((l64 & 3) | ((l64 >> 2) & 12));
    const int mf_h = (l64 >> 2) & 3;
    HadMfmaWords hw{};
    if constexpr (MF) hw = had_mfma_words(l64);
    const int64_t q_hs = a.q_hs, k_hs = a.k_hs, q_ts = a.q_ts, k_ts = a.k_ts;
    const int64_t v_hs = APPEND ? a.v_hs : 0, v_ts = APPEND ? a.v_ts : 0;
    const int hq = a.hq, hk = a.hk, H = a.hq + a.hk + (APPEND ? a.hv : 0);
    // Per-lane choices between argument fields select values, not addresses.
    const void* const qpost = HADR ? a.q_post : nullptr;
    const void* const kpost = HADR ? a.k_post : nullptr;
    const void* const vpost = HADR ? a.v_post : nullptr;
    char* const kcache = APPEND ? (char*)a.kc : nullptr;
    char* const vcache = APPEND ? (char*)a.vc : nullptr;
    const char* const qin = (const char*)a.q;
    const char* const kin = (const char*)a.k;
    const char* const vin = APPEND ? (const char*)a.v : nullptr;
    char* const qout = (char*)a.oq;
    char* const kout = (char*)a.ok;
    const int64_t oq_ts = QOUT ? a.oq_ts : q_ts, oq_hs = QOUT ? a.oq_hs : q_hs;
    const int R = a.R, R2 = a.R >> 1;
    using Item = NxItem<IO, NORM, SRC, P>;
    int64_t evaluated = -1;                   // SRC_FREQ: the token whose pairs the wave's LDS row holds
    // SRC_FREQ: the lane's rotary frequency inv_freq[l64], staged through LDS with the norm weights, so
    // that the item loop's only vector loads are the items' own (a wait for an evaluation's read of
    // inv_freq would also wait for the next item's loads).
    __shared__ float fsh[SRC == SRC_FREQ ? 64 : 1];
    float freq = 0.0f;

    // Loads of one item: the lane's two chunks of head (slice * P + p) * 8 + grp for each of the P passes,
    // and its rotary pairs (SRC_CS) or the token's position (SRC_FREQ).
    auto issue = [&](Item& t, int64_t item) __attribute__((always_inline)) {
        t.tok = (int64_t)udiv_magic((uint64_t)item, a.ns_m, a.ns_l);   // item / nslice
        t.slice = (int)(item - t.tok * nslice);
        // The row of head h of token tok.
        auto head_base = [&](int h) __attribute__((always_inline)) -> const char* {
            if constexpr (APPEND)
            {
                const bool iq = h < hq, iv = h >= hq + hk;
                const int hi = h - (iq ? 0 : hq) - (iv ? hk : 0);
                const int64_t ts = pick_qkv(iq, iv, q_ts, k_ts, v_ts), hs = pick_qkv(iq, iv, q_hs, k_hs, v_hs);
                return pick_qkv(iq, iv, qin, kin, vin) + (t.tok * ts + (int64_t)hi * hs) * IO::bytes;
            }
            else   // two choices: plain selects (the mask form costs this kernel ~0.5 us at C4)
                return h < hq ? qin + (t.tok * q_ts + (int64_t)h * q_hs) * IO::bytes
                              : kin + (t.tok * k_ts + (int64_t)(h - hq) * k_hs) * IO::bytes;
        };
        #pragma unroll
        for (int p = 0; p < P; ++p)
        {
            // Lanes past the last head take head H - 1: they load, compute and store exactly what that
            // head's lanes do (identical bytes to the same addresses), so every lane loads and stores
            // and no branch around a load or store makes the compiler's waits for the item's data cover
            // later loads too.
            if constexpr (MF)
            {
                // the two spans in had128_mfma's placement (lo: heads 0-3 of the pass, hi: heads 4-7)
                const int h0 = t.slice * 8 + mf_h;
                t.lo[p] = load8s<IO>(head_base(min(h0, H - 1)), mf_e);
                t.hi[p] = load8s<IO>(head_base(min(h0 + 4, H - 1)), mf_e);
            }
            else
            {
                const char* base = head_base(min((t.slice * P + p) * 8 + grp, H - 1));
                t.lo[p] = load8s<IO>(base, e0);
                t.hi[p] = load8s<IO>(base, e0 + 64);
            }
        }
        // The cache row, once per item that holds k or v heads (wave-uniform).
        if constexpr (APPEND) t.crow = (t.slice + 1) * 8 > hq ? cache_row_u(a, t.tok) : -1;
        if constexpr (SRC == SRC_CS)
        {
            // NeoX: pairs e0 .. e0 + 7; GPT-J: pairs e0/2 .. e0/2 + 3 (lo chunk) and 32 + e0/2 .. (hi chunk)
            const float2* row = a.cst + t.tok * R2;
            if constexpr (MODE == EXL3R_ROPE_NEOX)
            {
                #pragma unroll
                for (int i = 0; i < 4; ++i) t.cs[i] = ((const float4*)(row + e0))[i];
            }
            else
            {
                #pragma unroll
                for (int i = 0; i < 2; ++i)
                {
                    t.cs[i] = e0 / 2 + 2 * i < R2 ? ((const float4*)(row + e0 / 2))[i] : make_float4(0, 0, 0, 0);
                    t.cs[2 + i] = 32 + e0 / 2 + 2 * i < R2 ? ((const float4*)(row + 32 + e0 / 2))[i] : make_float4(0, 0, 0, 0);
                }
            }
        }
        else
            t.pos = token_position_u(a, t.tok);
    };

    if constexpr (NORM != NORM_NONE)
    {
        const int i = threadIdx.x, e = i & 127;
        const void* w = i < 128 ? a.qw : a.kw;
        if constexpr (NORM == NORM_HALF)
        {
            _Float16* wh = (_Float16*)wsh;
            wh[i] = w ? ((const _Float16*)w)[e] + to_f16(a.cb) : (_Float16)0.0f;
        }
        else
            wsh[i] = w ? load1(w, a.wt, e) + a.cb : 0.0f;
    }
    if constexpr (SRC == SRC_FREQ)
        if (threadIdx.x < 64) fsh[threadIdx.x] = (int)threadIdx.x < R2 ? a.inv_freq[threadIdx.x] : 0.0f;
    // HADR: the post-scales of all H heads (item-space order, 128 halfs each; zeros for a projection
    // without one, never read) into LDS after the {cos, sin} rows, 16 bytes per thread and step, so that
    // an item's read of them is an LDS read, whose wait does not also wait for the next item's loads.
    // (Indexed as an LDS array: a generic pointer into it trips an instruction-selection error in hipcc,
    // ROCm 7.2, for the comparisons of the flat address.)
    extern __shared__ u32x4 dyn16[];          // the dynamic LDS in 16-byte units
    constexpr int kPost16 = SRC == SRC_FREQ ? 4 * 64 * 8 / 16 : 0;
    if constexpr (HADR != HADR_NONE)
    {
        for (int i = threadIdx.x; i < H * 16; i += 256)
        {
            const int h = i >> 4;
            const bool iq = h < hq, iv = APPEND && h >= hq + hk;
            const int hi = h - (iq ? 0 : hq) - (iv ? hk : 0);
            const void* p = pick_qkv(iq, iv, qpost, kpost, vpost);
            u32x4 v = {};
            if (p) v = *(const u32x4*)((const _Float16*)p + (int64_t)hi * 128 + (i & 15) * 8);
            dyn16[kPost16 + i] = v;
        }
    }
    if constexpr (NORM != NORM_NONE || SRC == SRC_FREQ || HADR != HADR_NONE)
    {
        __syncthreads();
        if constexpr (SRC == SRC_FREQ) freq = fsh[l64];
    }

    // Head norm, rotation and stores of one pass (lo / hi: the lane's chunks of head h < H).
    auto pass = [&](int64_t tok, int h, typename IO::Vec& lo, typename IO::Vec& hi, const float (&c)[8],
                    const float (&s)[8], int64_t crow) __attribute__((always_inline)) {
        const bool isq = h < hq;
        const bool isv = APPEND && h >= hq + hk;
        const int hidx = h - (isq ? 0 : hq) - (isv ? hk : 0);
        if constexpr (HADR)
        {
            // The head's post-scale (f16 per column of the projection output), loaded before the
            // butterfly so that its latency hides under it (after it: 0.87x instead of 0.83x of the
            // wave-per-token kernel's time at C4), applied after its rounding.
            const void* post = pick_qkv(isq, isv, qpost, kpost, vpost);
            const bool hp = post != nullptr;
            u32x4 pl = {}, ph = {};
            auto load_post = [&]() __attribute__((always_inline)) {
                if (hp)
                {
                    pl = dyn16[kPost16 + h * 16 + (e0 >> 3)];
                    ph = dyn16[kPost16 + h * 16 + (e0 >> 3) + 8];
                }
            };
            if constexpr (!MF) load_post();
            if constexpr (MF)
            {
                // Both spans' MFMAs, one wait, the two lane stages and the rounding to f16 (exl3r_had_r_128_mfma's
                // operations on the same placement), then to the pass layout.
                MfmaOut m0, m1;
                had128_mfma_issue_w(hw, lo, hi, m0, m1);
                mfma_wait(m0, m1);
                float f[8];
                had128_mfma_finish(m0, f, l64, 0.0883883461356163f);
                lo = pack8<TF16>(f);
                had128_mfma_finish(m1, f, l64, 0.0883883461356163f);
                hi = pack8<TF16>(f);
                #pragma unroll
                for (int i = 0; i < 4; ++i)
                {
                    const auto w = __builtin_amdgcn_permlane32_swap((uint32_t)lo.a[i], (uint32_t)hi.a[i], false, false);
                    lo.a[i] = w[0];
                    hi.a[i] = w[1];
                }
                load_post();
            }
            else
                rotate_head_nx(lo, hi, l64 & 7);
            if (hp)
            {
                #pragma unroll
                for (int i = 0; i < 4; ++i)
                {
                    lo.a[i] = hmul2(lo.a[i], (uint32_t)pl[i]);
                    hi.a[i] = hmul2(hi.a[i], (uint32_t)ph[i]);
                }
            }
        }
        // v heads (APPEND) are only copied to the cache; a group of 8 lanes is one head, so the
        // head norm's exchanges stay inside lanes that take the same branch.
        if (!isv)
        {
        if constexpr (NORM != NORM_NONE)
        {
            float fl[8], fh[8];
            unpack8<IO>(lo, fl);
            unpack8<IO>(hi, fh);
            // fp64 sum of squares (as rope_head: exact for 16-bit data, one rounding to fp32)
            float mean;
            if (a.ss32)
            {
                float s32 = 0.0f;
                #pragma unroll
                for (int j = 0; j < 8; ++j) s32 = fmaf(fl[j], fl[j], s32);
                #pragma unroll
                for (int j = 0; j < 8; ++j) s32 = fmaf(fh[j], fh[j], s32);
                mean = nx_head_sum<HADR>(s32) * a.inv_hd;
            }
            else
            {
                double ss = 0.0;
                #pragma unroll
                for (int j = 0; j < 8; ++j) ss = fma((double)fl[j], (double)fl[j], ss);
                #pragma unroll
                for (int j = 0; j < 8; ++j) ss = fma((double)fh[j], (double)fh[j], ss);
                ss = nx_head_sum<HADR>(ss);
                mean = (float)ss * a.inv_hd;     // head_dim 128: an exact multiply
            }
            const float rmf = 1.0f / sqrtf(mean + a.eps);
            const int wo = (isq ? 0 : 128) + e0;
            if constexpr (NORM == NORM_HALF)
            {
                const u32x4 wl = *(const u32x4*)((const _Float16*)wsh + wo);
                const u32x4 wh = *(const u32x4*)((const _Float16*)wsh + wo + 64);
                #pragma unroll
                for (int i = 0; i < 4; ++i)
                {
                    const f16x2 nl = { to_f16(fl[2 * i] * rmf), to_f16(fl[2 * i + 1] * rmf) };
                    const f16x2 nh = { to_f16(fh[2 * i] * rmf), to_f16(fh[2 * i + 1] * rmf) };
                    // (uint32_t) first: a bit_cast of a single u32x4 element is lowered as a broadcast of
                    // element 0 by hipcc (ROCm 7.2) with the packed-fp32 forms disabled.
                    lo.a[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, (uint32_t)wl[i]) * nl);
                    hi.a[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, (uint32_t)wh[i]) * nh);
                }
            }
            else
            {
                // The product stays an fp32 value before the io rounding (opaque: no single-rounding
                // mixed multiply-convert).
                #pragma unroll
                for (int j = 0; j < 8; ++j)
                {
                    fl[j] = opaque((fl[j] * rmf) * wsh[wo + j]);
                    fh[j] = opaque((fh[j] * rmf) * wsh[wo + 64 + j]);
                }
                lo = pack8<IO>(fl);
                hi = pack8<IO>(fh);
            }
        }
        {
            // r1 = fl(fl(v1 c) - fl(v2 s)), r2 = fl(fl(v2 c) + fl(v1 s)), each rounded once to io.
            #pragma clang fp contract(off)
            if constexpr (MODE == EXL3R_ROPE_NEOX && IO::code == DT_F16)
            {
                // The products straight from the packed f16 pairs (no unpacking; the same roundings).
                float fl[8], fh[8];
                #pragma unroll
                for (int i = 0; i < 4; ++i)
                {
                    const uint32_t x = lo.a[i], y = hi.a[i];
                    fl[2 * i] = opaque(mul_f16_f32<false>(x, c[2 * i]) - mul_f16_f32<false>(y, s[2 * i]));
                    fh[2 * i] = opaque(mul_f16_f32<false>(y, c[2 * i]) + mul_f16_f32<false>(x, s[2 * i]));
                    fl[2 * i + 1] = opaque(mul_f16_f32<true>(x, c[2 * i + 1]) - mul_f16_f32<true>(y, s[2 * i + 1]));
                    fh[2 * i + 1] = opaque(mul_f16_f32<true>(y, c[2 * i + 1]) + mul_f16_f32<true>(x, s[2 * i + 1]));
                }
                lo = pack8<IO>(fl);
                hi = pack8<IO>(fh);
            }
            else if constexpr (IO::code == DT_F16)
            {
                // GPT-J f16: a pair is the two halves of one packed word, its products taken from the word;
                // dims >= rotary_dim keep their bits.  c / s [0, 4): the lo chunk's pairs, [4, 8): the hi chunk's.
                auto pair = [](uint32_t w, float cc, float ss) __attribute__((always_inline)) {
                    const float r1 = opaque(mul_f16_f32<false>(w, cc) - mul_f16_f32<true>(w, ss));
                    const float r2 = opaque(mul_f16_f32<true>(w, cc) + mul_f16_f32<false>(w, ss));
                    return pack_f16(r1, r2);
                };
                #pragma unroll
                for (int i = 0; i < 4; ++i)
                {
                    if (e0 + 2 * i < R) lo.a[i] = pair(lo.a[i], c[i], s[i]);
                    if (64 + e0 + 2 * i < R) hi.a[i] = pair(hi.a[i], c[4 + i], s[4 + i]);
                }
            }
            else
            {
                float fl[8], fh[8];
                unpack8<IO>(lo, fl);
                unpack8<IO>(hi, fh);
                if constexpr (MODE == EXL3R_ROPE_NEOX)
                {
                    #pragma unroll
                    for (int j = 0; j < 8; ++j)
                    {
                        const float x = fl[j], y = fh[j];
                        fl[j] = opaque(x * c[j] - y * s[j]);
                        fh[j] = opaque(y * c[j] + x * s[j]);
                    }
                }
                else
                {
                    // c / s [0, 4): the lo chunk's pairs, [4, 8): the hi chunk's; dims >= rotary_dim pass through
                    #pragma unroll
                    for (int i = 0; i < 4; ++i)
                    {
                        if (e0 + 2 * i < R)
                        {
                            const float x = fl[2 * i], y = fl[2 * i + 1];
                            fl[2 * i] = opaque(x * c[i] - y * s[i]);
                            fl[2 * i + 1] = opaque(y * c[i] + x * s[i]);
                        }
                        if (64 + e0 + 2 * i < R)
                        {
                            const float x = fh[2 * i], y = fh[2 * i + 1];
                            fh[2 * i] = opaque(x * c[4 + i] - y * s[4 + i]);
                            fh[2 * i + 1] = opaque(y * c[4 + i] + x * s[4 + i]);
                        }
                    }
                }
                lo = pack8<IO>(fl);
                hi = pack8<IO>(fh);
            }
        }
        }
        if (isq || (!isv && (!APPEND || kout)))
        {
            char* ob;
            int32_t oo;
            if (isq)
            {
                ob = qout + tok * oq_ts * IO::bytes;
                oo = (int32_t)((int64_t)h * oq_hs) + e0;
            }
            else
            {
                ob = kout + tok * k_ts * IO::bytes;
                oo = (int32_t)((int64_t)hidx * k_hs) + e0;
            }
            store8<IO>(ob, oo, lo);
            store8<IO>(ob, oo + 64, hi);
        }
        if constexpr (APPEND)
        {
            if (!isq && crow >= 0)
            {
                char* cb = isv ? vcache : kcache;
                const int64_t co = crow + (int64_t)hidx * 128 + e0;
                store8<IO>(cb, co, lo);
                store8<IO>(cb, co + 64, hi);
            }
        }
    };

    auto compute = [&](Item& t) __attribute__((always_inline)) {
        float c[8], s[8];
        if constexpr (SRC == SRC_CS)
        {
            #pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                c[2 * i] = t.cs[i].x;
                s[2 * i] = t.cs[i].y;
                c[2 * i + 1] = t.cs[i].z;
                s[2 * i + 1] = t.cs[i].w;
            }
        }
        else
        {
            float2* row = cs + wave * 64;
            if (t.tok != evaluated)           // wave-uniform: once per token within a run
            {
                wave_lds_sync();
                if (MODE == EXL3R_ROPE_NEOX || l64 < R2) row[l64] = rope_cs_of_angle(__fmul_rn(freq, (float)t.pos), a.attn);
                wave_lds_sync();
                evaluated = t.tok;
            }
            #pragma unroll
            for (int j = 0; j < 8; ++j)
            {
                // NeoX: pair e0 + j; GPT-J: pair e0/2 + j (lo chunk, j < 4) or 32 + e0/2 + j - 4 (hi chunk)
                const int tp = MODE == EXL3R_ROPE_NEOX ? e0 + j : j < 4 ? e0 / 2 + j : 32 + e0 / 2 + (j - 4);
                const float2 x = MODE == EXL3R_ROPE_NEOX || tp < R2 ? row[tp] : make_float2(0.0f, 0.0f);   // NeoX: R2 = 64
                c[j] = x.x;
                s[j] = x.y;
            }
        }
        #pragma unroll
        for (int p = 0; p < P; ++p)
            if (p == 0 || (t.slice * P + p) * 8 < H)   // wave-uniform: a pass past the last head is skipped whole
                pass(t.tok, min((t.slice * P + p) * 8 + grp, H - 1), t.lo[p], t.hi[p], c, s, APPEND ? t.crow : -1);
    };

    int64_t item = ((int64_t)blockIdx.x * 4 + wave) * run;
    if (item >= items) return;
    int j = 0;                                // item's place in its run
    auto next = [&](int64_t it) __attribute__((always_inline)) -> int64_t {
        if (++j < run) return it + 1;
        j = 0;
        return it + 1 + (W - 1) * run;
    };
    // Issue the next item's loads, then finish this one (the loop alternates the two buffers).  (The
    // compiler's wait for an item's data also covers the next item's loads, the issue being conditional;
    // finishing each wave's last item on a path of its own makes that wait exact, but the second copy of
    // the item code costs registers and measured no faster: C4 32.6 us either way, from the table 33.2
    // against 31.2 us.  An unconditional issue -- past its last item a wave reloading the grid's last
    // item -- makes it exact too (vmcnt(2) instead of vmcnt(0) before an item's math) and ran slower in
    // every instance, same process: C4 33.1 -> 33.9 us, from the table 31.4 -> 39.3, the rotating paged
    // form 38.4 -> 58.4 (13-20 VGPRs spilled: the next item's registers live across the math).  Issuing
    // the first item before the setup barrier ran the same or slower (the rotating C4 form 38.7 -> 41.4
    // us: 3 VGPRs spilled), and so did carrying the item's token / slice along the walk instead of
    // dividing (plain C4 at 93 VGPRs instead of 85).)
    Item A, B;
    issue(A, item);
    for (;;)
    {
        const int64_t nb = next(item);
        if (nb < items) issue(B, nb);
        compute(A);
        if (nb >= items) break;
        const int64_t na = next(nb);
        if (na < items) issue(A, na);
        compute(B);
        if (na >= items) break;
        item = na;
    }
}

// The k_rope_nx launch: head_dim 128 at prefill sizes (NeoX with rotary_dim 128, GPT-J with rotary_dim a
// multiple of 4), from inv_freq or a 16-byte aligned {cos, sin} table (no angle table), plain, with the
// paged append, and / or with the output rotations (16-byte aligned post-scales).  The grid walks the
// items with the workgroups resident at once.
// had: the launch carries the output rotations (exl3r_rope_had, exl3r_rope_paged_kv_had).
static bool rope_nx_ok(const RopeArgs& a, int rope_mode, bool had = false)
{
    const Tuning& tu = tuning();
    auto a16 = [](const void* p) { return p == nullptr || aligned16(p); };
    // GPT-J: rotary_dim % 4 == 0 keeps each 16-byte table read (two pairs) inside the token's row.
    if (tu.rope_nx < 0 || a.hd != 128 || (rope_mode == EXL3R_ROPE_NEOX ? a.R != 128 : a.R % 4 != 0) || a.table)
        return false;
    if (tu.rope_tok != 0 && tu.rope_nx == 0) return false;   // a test forcing one of the other kernels
    if (a.kc && a.hv != a.hk) return false;
    // the output rotations' post-scales of all heads in LDS: up to 192 heads (48 KB)
    if (had && (int64_t)(a.hq + a.hk + (a.kc ? a.hv : 0)) * 256 > (48 << 10)) return false;
    if (a.tokens >= ((int64_t)1 << 31)) return false;    // 32-bit token arithmetic
    if (!a16(a.q_post) || !a16(a.k_post) || !a16(a.v_post)) return false;
    if (a.cst && ((uintptr_t)a.cst & 15)) return false;
    // Every size: at decode and small prefills too it beats the flattened kernel (MI355X, HIP graph,
    // 64 / 8 heads, us: 1 token 3.21 vs 3.31, 64 tokens 3.51 vs 3.87, 256 tokens 4.60 vs 5.38; 512 tokens
    // of 16 / 8 heads 4.00 vs 4.36, of 64 / 8 heads 5.87 vs 7.69).
    return true;
}

template <class IO, int MODE, int NORM, int SRC, bool QOUT, int P, bool APPEND = false, int HADR = HADR_NONE>
static void launch_rope_nx_p(const RopeArgs& a, hipStream_t s)
{
    const int H = a.hq + a.hk + (APPEND ? a.hv : 0);
    const int nslice = ((H + 7) / 8 + P - 1) / P;
    const int64_t items = a.tokens * nslice;
    // The output rotations' post-scales sit in LDS (H * 256 bytes; rope_nx_ok bounds H).  Up to 96 heads
    // five workgroups of 20 resident waves per CU take at most 130 KB of its 160 KB with the {cos, sin}
    // rows; more heads can lower the occupancy, which is then asked for at the launch.
    const size_t cs_lds = SRC == SRC_FREQ ? 4 * 64 * sizeof(float2) : 0;
    const size_t lds = cs_lds + (HADR != HADR_NONE ? (size_t)H * 256 : 0);
    constexpr size_t kLdsCommon = SRC == SRC_FREQ ? 4 * 64 * sizeof(float2) + (HADR != HADR_NONE ? 24 << 10 : 0)
                                                  : (HADR != HADR_NONE ? 24 << 10 : 0);
    // Grid: the workgroups resident at once (per CU, from the occupancy of this instance), each wave
    // walking its items i, i + W, ...
    auto occupancy = [](size_t bytes) {
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_rope_nx<IO, MODE, NORM, SRC, QOUT, P, APPEND, HADR>, 256,
                                                         bytes) != hipSuccess || nb < 1)
            nb = 4;
        return nb;
    };
    static const int resident_common = occupancy(kLdsCommon);   // per template instance; thread-safe init
    const int resident = lds <= kLdsCommon ? resident_common : occupancy(lds);
    const int wpc = tuning().rope_wgs_per_cu;
    int64_t blocks = (int64_t)(wpc > 0 ? wpc : resident) * device_cus();
    // Items a wave takes in a row, its token's angles evaluated once within them, where every wave gets
    // whole runs (prefill sizes).  MI355X, same process, us at runs of 1 / 2 / 3: C4 NeoX 33.2 / 32.1 /
    // 33.3; q / k rotations + RoPE at C4 46.8 / 45.5 / 42.7; q / k / v rotations + RoPE + paged append at
    // 4096 tokens 57.5 / 53.4 / 51.3, from the {cos, sin} table 48.4 / 47.1 / 46.1 (the post-scales and
    // cache rows of one token reused too).  Two passes per item (GPT-J) and the plain kernel reading the
    // table are fastest at 1.  q / k norm + RoPE + paged append at 4096 tokens, runs of 1 / 2 / 3 / 4 / 6:
    // 42.5 / 38.8 / 39.7 / 38.5 / 39.6, from the table 38.2 / 36.5 / 38.3 / 35.8 / 41.3 (the wave-per-token
    // kernel: 41.7 / 38.8).  The q | g split (rope_qg, Qwen3.5 4096 tokens) at runs of 1 / 2 / 4: 35.4 /
    // 34.7 / 34.5.
    constexpr int kRun = HADR ? 3 : APPEND ? 4 : SRC == SRC_FREQ && P == 1 ? 2 : 1;
    const int tr = tuning().rope_nx_run;
    const int run = tr > 0 ? tr : items >= (int64_t)kRun * blocks * 4 ? kRun : 1;
    const int64_t runs = (items + run - 1) / run;
    // Plain passes reading the {cos, sin} table carry nothing from one item to the next: a wave per
    // run over the whole grid, dispatched as workgroups retire, beats the resident grid (C4, same
    // process: 30.8 vs 32.1 us; the evaluated and the GPT-J passes lose with it, 37.5 / 35.7 us).
    constexpr bool kFlat = SRC == SRC_CS && P == 1 && !APPEND && !HADR;
    if (kFlat && wpc == 0) blocks = (runs + 3) / 4;
    if (blocks > (runs + 3) / 4) blocks = (runs + 3) / 4;
    if (blocks > kMaxGridX) blocks = kMaxGridX;
    RopeArgs b = a;
    udiv_magic_init((uint64_t)nslice, b.ns_m, b.ns_l);
    launch(k_rope_nx<IO, MODE, NORM, SRC, QOUT, P, APPEND, HADR>, (unsigned)blocks, 256, lds, s, b, nslice, run);
}

// Passes per item: one for NeoX, two for GPT-J (its token's sin / cos or table row shared by two passes).
// MI355X, C4 f16, 10 interleaved windows on one box (us, one / two passes / the wave-per-token or flattened
// kernel): NeoX evaluated 32.9 / 33.9 / 38.1, from the table 31.7 / 32.9 / 36.4, GPT-J 35.4 / 34.9 / 35.3;
// Qwen3.5 q | g split 36.4 / 36.6 / 37.4.
template <class IO, int MODE, int NORM, int SRC, bool QOUT>
static void launch_rope_nx(const RopeArgs& a, hipStream_t s)
{
    if constexpr (!QOUT)
    {
        if (a.kc)
        {
            launch_rope_nx_p<IO, MODE, NORM, SRC, false, 1, true>(a, s);
            return;
        }
    }
    const int tp = tuning().rope_nx;
    if (tp == 2 || (tp == 0 && MODE == EXL3R_ROPE_GPTJ && !QOUT && a.tokens >= 1024))
        launch_rope_nx_p<IO, MODE, NORM, SRC, QOUT, 2>(a, s);
    else launch_rope_nx_p<IO, MODE, NORM, SRC, QOUT, 1>(a, s);
}

// The output rotations (exl3r_rope_had, exl3r_rope_paged_kv_had) in the 8-lane kernel, f16 heads: on the
// matrix cores, or (exact) as the reference's butterfly.
template <int NORM>
static void launch_had_nx(const RopeArgs& a, int rope_mode, bool exact, hipStream_t s)
{
    auto go = [&](auto M, auto X) {
        constexpr int MODE = decltype(M)::value, HADR = decltype(X)::value;
        if (a.kc)
        {
            if (a.cst) launch_rope_nx_p<TF16, MODE, NORM, SRC_CS, false, 1, true, HADR>(a, s);
            else launch_rope_nx_p<TF16, MODE, NORM, SRC_FREQ, false, 1, true, HADR>(a, s);
        }
        else if (a.cst) launch_rope_nx_p<TF16, MODE, NORM, SRC_CS, false, 1, false, HADR>(a, s);
        else launch_rope_nx_p<TF16, MODE, NORM, SRC_FREQ, false, 1, false, HADR>(a, s);
    };
    auto with_mode = [&](auto X) {
        if (rope_mode == EXL3R_ROPE_GPTJ) go(std::integral_constant<int, EXL3R_ROPE_GPTJ>{}, X);
        else go(std::integral_constant<int, EXL3R_ROPE_NEOX>{}, X);
    };
    if (exact) with_mode(std::integral_constant<int, HADR_EXACT>{});
    else with_mode(std::integral_constant<int, HADR_MFMA>{});
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
    fill_sincos(a, (int)tok, token_position(a, (int)tok), cs);
    const int64_t crow = a.kc ? cache_row(a, tok) : -1;
    __syncthreads();
    for (int head = 0; head < a.hq + a.hk + a.hv; ++head)
    {
        const int kind = head_kind(a, head);
        const bool isq = kind == KIND_Q;
        const int hkv = head - a.hq - (kind == KIND_V ? a.hk : 0);
        const void* ip = isq ? a.q : kind == KIND_K ? a.k : a.v;
        void* op = isq ? a.oq : kind == KIND_K ? a.ok : nullptr;
        const int64_t off = isq ? tok * a.q_ts + (int64_t)head * a.q_hs
                                : kind == KIND_K ? tok * a.k_ts + (int64_t)hkv * a.k_hs : tok * a.v_ts + (int64_t)hkv * a.v_hs;
        const int64_t ooff = isq ? tok * a.oq_ts + (int64_t)head * a.oq_hs : off;
        void* cp = crow >= 0 && kind != KIND_Q ? (kind == KIND_K ? a.kc : a.vc) : nullptr;
        const int64_t coff = crow + (int64_t)hkv * a.hd;
        if (kind == KIND_V)
        {
            for (int d = tid; d < a.hd; d += blockDim.x)
                if (cp) store1(cp, dt, coff + d, load1(ip, dt, off + d));
            continue;
        }
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
        for (int d = tid; d < a.hd; d += blockDim.x)
        {
            if (op) store1(op, dt, ooff + d, hv[d]);
            if (cp) store1(cp, dt, coff + d, hv[d]);
        }
        __syncthreads();
    }
    }
}

template <class IO, int MODE, int LPH, int NORM, int SRC>
static void launch_rope_lph(RopeArgs a, int iters, hipStream_t s)
{
    const int threads = 256;
    const int64_t per_wg = (int64_t)(threads / LPH) * iters;
    const int nheads = a.hq + a.hk + a.hv;
    a.tok_span = (int)((nheads + per_wg - 2) / nheads) + 1;
    const int64_t items = a.tokens * nheads;
    int64_t blocks = (items + per_wg - 1) / per_wg;
    if (blocks > kMaxGridX) blocks = kMaxGridX;
    const size_t lds = (size_t)a.tok_span * (a.R / 2) * sizeof(float2);
    if constexpr (SRC != SRC_FREQ)
    {
        // Angle tables (never with a paged append) and {cos, sin} tables: two heads per lane.
        if constexpr (SRC == SRC_CS)
        {
            if (a.kc)
            {
                launch(k_rope<IO, MODE, LPH, 2, NORM, true, SRC>, (unsigned)blocks, threads, lds, s, a);
                return;
            }
        }
        launch(k_rope<IO, MODE, LPH, 2, NORM, false, SRC>, (unsigned)blocks, threads, lds, s, a);
        return;
    }
    auto go = [&](auto I) {
        constexpr int IT = decltype(I)::value;
        if (a.kc) launch(k_rope<IO, MODE, LPH, IT, NORM, true, SRC_FREQ>, (unsigned)blocks, threads, lds, s, a);
        else launch(k_rope<IO, MODE, LPH, IT, NORM, false, SRC_FREQ>, (unsigned)blocks, threads, lds, s, a);
    };
    switch (iters)
    {
        case 1: go(std::integral_constant<int, 1>{}); break;
        case 2: go(std::integral_constant<int, 2>{}); break;
        default: go(std::integral_constant<int, 4>{}); break;
    }
}

// Wave-per-token launch.  Measured on MI355X at C4 (4639 tokens, 64 + 8 heads of 128, NeoX, in
// place): f16 heads (packed-half norm, 94 VGPRs) run best with 2 heads per lane in flight and one
// token per wave (38.5 us; 3 per lane 42 us); bf16 heads (fp32 norm) with 3 per lane on a
// persistent grid of 4 workgroups per CU (37.0 us; 2 per lane 42 us).  With the paged append
// (4096 tokens, + 8 v heads) 3 per lane: 40.0 us, 2 per lane 41-43 us.
template <class IO, int MODE, int LPH, int NORM, bool HADR = false, int SRC = SRC_FREQ, bool QOUT = false>
static void launch_rope_tok(RopeArgs a, hipStream_t s)
{
    const Tuning& tu = tuning();
    // With the output rotation (HADR; C4 shape: 62.1 us against 66.6 us with the plain kernel's
    // shape) the kernel takes the bf16 shape: 3 heads per lane, 4 workgroups per CU.
    int hpl = IO::code == DT_F16 && !a.kc && !HADR ? 2 : 3;
    int wgs_per_cu = IO::code == DT_F16 && !HADR ? 0 : 4;
    if (tu.rope_hpl > 0) hpl = tu.rope_hpl;
    if (tu.rope_wgs_per_cu > 0) wgs_per_cu = tu.rope_wgs_per_cu;
    hpl = hpl <= 2 ? 2 : 3;
    int64_t blocks = (a.tokens + 3) / 4;
    if (wgs_per_cu > 0 && blocks > (int64_t)wgs_per_cu * device_cus()) blocks = (int64_t)wgs_per_cu * device_cus();
    if (blocks > kMaxGridX) blocks = kMaxGridX;
    const size_t lds = 4 * (size_t)(a.R / 2) * sizeof(float2);
    auto go = [&](auto H) {
        constexpr int HP = decltype(H)::value;
        if constexpr (QOUT)
            launch(k_rope_tok<IO, MODE, LPH, HP, NORM, false, false, SRC_FREQ, true>, (unsigned)blocks, 256, lds, s, a);
        else if (a.kc) launch(k_rope_tok<IO, MODE, LPH, HP, NORM, true, HADR, SRC>, (unsigned)blocks, 256, lds, s, a);
        else launch(k_rope_tok<IO, MODE, LPH, HP, NORM, false, HADR, SRC>, (unsigned)blocks, 256, lds, s, a);
    };
    if (hpl == 2) go(std::integral_constant<int, 2>{});
    else go(std::integral_constant<int, 3>{});
}

static bool rope_tok_launch(const RopeArgs& a);

// Prefill-sized NeoX launches (a wave per token still gives every CU several waves) take the
// wave-per-token kernel.  GPT-J (C4 at rotary 64: 35.2 us flattened vs 37.5 us per token) and
// decode-sized launches take the flattened kernel: items per lane enough workgroups to fill 256 CUs
// several times over, then up to four heads per lane so each wave keeps 4 KiB of loads in flight.
template <class IO, int MODE, int NORM>
static void launch_rope_vec(const RopeArgs& a, int lph, hipStream_t s)
{
    const Tuning& tu = tuning();
    if (rope_nx_ok(a, MODE))
    {
        const bool qout = a.oq_ts != a.q_ts || a.oq_hs != a.q_hs;
        if (a.cst) launch_rope_nx<IO, MODE, NORM, SRC_CS, false>(a, s);
        else if (qout) launch_rope_nx<IO, MODE, NORM, SRC_FREQ, true>(a, s);
        else launch_rope_nx<IO, MODE, NORM, SRC_FREQ, false>(a, s);
        return;
    }
    if (a.cst)
    {
        // A {cos, sin} table (exl3r_rope_cs, or the cs_table of the paged / rotating entries): the
        // kernels of exl3r_rope, which copy the token's table row to LDS in place of evaluating it.
        if (MODE == EXL3R_ROPE_NEOX && rope_tok_launch(a))
        {
            if (lph == 8) launch_rope_tok<IO, MODE, 8, NORM, false, SRC_CS>(a, s);
            else if (lph == 16) launch_rope_tok<IO, MODE, 16, NORM, false, SRC_CS>(a, s);
            else launch_rope_tok<IO, MODE, 32, NORM, false, SRC_CS>(a, s);
        }
        else if (lph == 8) launch_rope_lph<IO, MODE, 8, NORM, SRC_CS>(a, 2, s);
        else if (lph == 16) launch_rope_lph<IO, MODE, 16, NORM, SRC_CS>(a, 2, s);
        else launch_rope_lph<IO, MODE, 32, NORM, SRC_CS>(a, 2, s);
        return;
    }
    if (a.table)
    {
        if (lph == 8) launch_rope_lph<IO, MODE, 8, NORM, SRC_ANGLE>(a, 2, s);
        else if (lph == 16) launch_rope_lph<IO, MODE, 16, NORM, SRC_ANGLE>(a, 2, s);
        else launch_rope_lph<IO, MODE, 32, NORM, SRC_ANGLE>(a, 2, s);
        return;
    }
    if constexpr (MODE == EXL3R_ROPE_NEOX)
    {
        if (rope_tok_launch(a) && (a.oq_ts != a.q_ts || a.oq_hs != a.q_hs))
        {
            // exl3r_rope_qg (no append): out_q in its own layout.
            if (lph == 8) launch_rope_tok<IO, MODE, 8, NORM, false, SRC_FREQ, true>(a, s);
            else if (lph == 16) launch_rope_tok<IO, MODE, 16, NORM, false, SRC_FREQ, true>(a, s);
            else launch_rope_tok<IO, MODE, 32, NORM, false, SRC_FREQ, true>(a, s);
            return;
        }
        if (rope_tok_launch(a))
        {
            if (lph == 8) launch_rope_tok<IO, MODE, 8, NORM>(a, s);
            else if (lph == 16) launch_rope_tok<IO, MODE, 16, NORM>(a, s);
            else launch_rope_tok<IO, MODE, 32, NORM>(a, s);
            return;
        }
    }
    const int64_t items = a.tokens * (a.hq + a.hk + a.hv);
    const int64_t slots = 256 / lph;
    int iters = 1;
    if (tu.rope_iters == 1 || tu.rope_iters == 2 || tu.rope_iters == 4) iters = tu.rope_iters;
    else if (items >= slots * 4 * 2048) iters = 4;
    else if (items >= slots * 2 * 2048) iters = 2;
    if (lph == 8) launch_rope_lph<IO, MODE, 8, NORM, SRC_FREQ>(a, iters, s);
    else if (lph == 16) launch_rope_lph<IO, MODE, 16, NORM, SRC_FREQ>(a, iters, s);
    else launch_rope_lph<IO, MODE, 32, NORM, SRC_FREQ>(a, iters, s);
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

// Argument checks and RopeArgs of the rotary part, shared by exl3r_rope and exl3r_rope_paged_kv.
// Returns EXL3R_OK with a.tokens == 0 when there is nothing to launch.
static int rope_prepare(const char* op, RopeArgs& a, const void* q, void* out_q, int64_t q_tok_stride,
                        int64_t q_head_stride, int num_heads_q, const void* k, void* out_k, bool out_k_optional,
                        int64_t k_tok_stride, int64_t k_head_stride, int num_heads_k, int dtype, int64_t bsz,
                        int64_t seq_len, int head_dim, const float* inv_freq, int rotary_dim, int32_t position,
                        const int32_t* positions, const int32_t* position_ids, const void* q_norm, const void* k_norm,
                        int norm_dtype, float norm_eps, float norm_constant_bias, int rope_mode, float attn_factor)
{
    if (!inv_freq) return set_error(EXL3R_EINVAL, "%s: inv_freq (angle table) must be non-null", op);
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
    if (k && ((bsz * seq_len > 0 && !out_k && !out_k_optional) || k_head_stride < head_dim ||
              k_tok_stride < (int64_t)num_heads_k * k_head_stride))
        return set_error(EXL3R_EINVAL, "%s: k needs out_k and non-overlapping strides", op);
    if (positions && position_ids) return set_error(EXL3R_EINVAL, "%s: at most one of positions / position_ids", op);
    if (q_norm && k && !k_norm) return set_error(EXL3R_EINVAL, "%s: q_norm given without k_norm", op);
    if (!q_norm && k_norm) return set_error(EXL3R_EINVAL, "%s: k_norm given without q_norm", op);
    if (q_norm && !is_float_dtype(norm_dtype))
        return set_error(EXL3R_EDTYPE, "%s: unsupported norm weight dtype %s", op, dtype_name(norm_dtype));
    const int64_t tokens = bsz * seq_len;
    a = RopeArgs{};
    if (tokens == 0) return EXL3R_OK;
    if (!q || !out_q) return set_error(EXL3R_EINVAL, "%s: q and out_q must be non-null", op);
    if (tokens > 0x7fffffff) return set_error(EXL3R_EINVAL, "%s: too many tokens", op);

    a.q = q; a.oq = out_q; a.k = k; a.ok = out_k;
    a.q_ts = q_tok_stride; a.q_hs = q_head_stride; a.k_ts = k_tok_stride; a.k_hs = k_head_stride;
    a.oq_ts = q_tok_stride; a.oq_hs = q_head_stride;
    a.hq = num_heads_q; a.hk = k ? num_heads_k : 0; a.hd = head_dim; a.R = rotary_dim;
    a.seq_len = seq_len; a.tokens = tokens; a.inv_freq = inv_freq;
    a.position = position; a.positions = positions; a.position_ids = position_ids;
    a.qw = q_norm; a.kw = k_norm; a.wt = norm_dtype;
    a.eps = norm_eps; a.cb = norm_constant_bias; a.attn = attn_factor;
    a.inv_hd = (head_dim & (head_dim - 1)) == 0 ? 1.0f / (float)head_dim : 0.0f;
#ifdef EXL3R_TUNING
    a.ss32 = tuning().rope_ss32;
#endif
    return EXL3R_OK;
}

// Precomputed {cos, sin} * attn_factor (exl3r_rope_cs_table): row tok of [tokens, R / 2] holds the
// rotary pairs of token tok's position, evaluated as rope_cs does, so RoPE from the table is
// bit-identical to RoPE that evaluates them itself.
__global__ __launch_bounds__(256) void k_rope_cs_table(RopeArgs a, float2* cst)
{
    const int R2 = a.R >> 1;
    const int64_t n = a.tokens * R2;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    {
        const int64_t tok = i / R2;
        const int t = (int)(i - tok * R2);
        cst[i] = rope_cs<SRC_FREQ>(a, t, (int)tok, token_position(a, (int)tok));
    }
}

static int rope_norm_kind(const RopeArgs& a, int dtype)
{
    return !a.qw ? NORM_NONE : (a.wt == EXL3R_F16 && dtype == EXL3R_F16) ? NORM_HALF : NORM_F32;
}

static int rope_lph(const RopeArgs& a)
{
    int lph = 1;
    while (lph * 8 < a.hd) lph *= 2;
    return lph;
}

// Vector kernels: 8-element lane chunks, 8 to 32 lanes per head (head_dim 64 .. 256), 16-byte
// aligned rows and heads.
static bool rope_vec_ok(const RopeArgs& a, int rope_mode)
{
    auto a16 = [](const void* p) { return p == nullptr || aligned16(p); };
    const int lph = rope_lph(a);
    bool vec = a.hd % 8 == 0 && lph >= 8 && lph <= 32 && a.R % (rope_mode == EXL3R_ROPE_NEOX ? 16 : 2) == 0;
    vec = vec && aligned16(a.q) && aligned16(a.oq) && a.q_ts % 8 == 0 && a.q_hs % 8 == 0;
    vec = vec && a.oq_ts % 8 == 0 && a.oq_hs % 8 == 0;
    vec = vec && (!a.k || (aligned16(a.k) && a16(a.ok) && a.k_ts % 8 == 0 && a.k_hs % 8 == 0));
    vec = vec && (!a.v || (aligned16(a.v) && a.v_ts % 8 == 0 && a.v_hs % 8 == 0 && a16(a.kc) && a16(a.vc)));
    vec = vec && (!a.qw || (aligned16(a.qw) && a16(a.kw)));
    return vec;
}

// Prefill-sized NeoX launches take the wave-per-token kernel (launch_rope_vec).
static bool rope_tok_launch(const RopeArgs& a)
{
    const Tuning& tu = tuning();
    return tu.rope_tok == 2 || (tu.rope_tok == 0 && a.tokens >= 1024);
}

static int rope_dispatch(const char* op, const RopeArgs& a, int dtype, int rope_mode, void* stream)
{
    const int norm = rope_norm_kind(a, dtype);
    hipStream_t s = (hipStream_t)stream;
    const int lph = rope_lph(a);
    if (rope_vec_ok(a, rope_mode))
    {
        if (dtype == EXL3R_F16) launch_rope_io<TF16>(a, rope_mode, norm, lph, s);
        else launch_rope_io<TBF16>(a, rope_mode, norm, lph, s);
    }
    else
    {
        const size_t lds = (size_t)(a.R / 2) * sizeof(float2) + (size_t)a.hd * sizeof(float);
        launch(k_rope_generic, (unsigned)(a.tokens < kMaxGridX ? a.tokens : kMaxGridX), 256, lds, s, a, dtype, rope_mode, norm);
    }
    return launch_status(op);
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
    begin_call();
    const char* op = "exl3r_rope";
    RopeArgs a;
    const int rc = rope_prepare(op, a, q, out_q, q_tok_stride, q_head_stride, num_heads_q, k, out_k, false, k_tok_stride,
                                k_head_stride, num_heads_k, dtype, bsz, seq_len, head_dim, inv_freq, rotary_dim, position,
                                positions, position_ids, q_norm, k_norm, norm_dtype, norm_eps, norm_constant_bias,
                                rope_mode, attn_factor);
    if (rc || a.tokens == 0) return rc;
    return rope_dispatch(op, a, dtype, rope_mode, stream);
}

// The optional {cos, sin} table of the paged and rotating entry points (built by exl3r_rope_cs_table for
// the same positions): the kernels read it in place of evaluating sin / cos from inv_freq.
static int use_cs_table(const char* op, RopeArgs& a, const void* cs_table)
{
    if (!cs_table) return EXL3R_OK;
    if ((uintptr_t)cs_table % 8) return set_error(EXL3R_EINVAL, "%s: cs_table must be 8-byte aligned", op);
    a.cst = (const float2*)cs_table;
    a.inv_freq = nullptr;
    return EXL3R_OK;
}

// The rotation source rope_prepare checks: inv_freq, or the cs_table standing in for it.
static const float* rotation_source(const float* inv_freq, const void* cs_table)
{
    return inv_freq ? inv_freq : (const float*)cs_table;
}

// Launches the wave-per-token kernel with the output rotation, the rotary pairs evaluated or read
// from the {cos, sin} table.
template <int NORM>
static void launch_had_tok(const RopeArgs& a, hipStream_t s)
{
    if (a.cst) launch_rope_tok<TF16, EXL3R_ROPE_NEOX, 16, NORM, true, SRC_CS>(a, s);
    else launch_rope_tok<TF16, EXL3R_ROPE_NEOX, 16, NORM, true>(a, s);
}

// Argument checks and RopeArgs of the fused append, shared by exl3r_rope_paged_kv and
// exl3r_rope_paged_kv_had.  Returns EXL3R_OK with a.tokens == 0 when there is nothing to launch.
static int paged_prepare(const char* op, RopeArgs& a, const void* q, void* out_q, int64_t q_tok_stride,
                         int64_t q_head_stride, int num_heads_q, const void* k, void* out_k, int64_t k_tok_stride,
                         int64_t k_head_stride, const void* v, int64_t v_tok_stride, int64_t v_head_stride,
                         int num_heads_kv, int dtype, int64_t bsz, int64_t seq_len, int head_dim,
                         const float* inv_freq, int rotary_dim, int32_t position, const int32_t* positions,
                         const int32_t* position_ids, const void* q_norm, const void* k_norm, int norm_dtype,
                         float norm_eps, float norm_constant_bias, int rope_mode, float attn_factor,
                         void* k_cache, void* v_cache, int page_size, int64_t num_pages,
                         const int32_t* block_table, int64_t max_blocks_per_seq, const int32_t* cache_seqlens,
                         int32_t* err_flag)
{
    if (num_heads_kv <= 0) return set_error(EXL3R_EINVAL, "%s: num_heads_kv must be positive", op);
    if (page_size <= 0 || (page_size & (page_size - 1)) || num_pages <= 0 || max_blocks_per_seq <= 0)
        return set_error(EXL3R_EINVAL, "%s: page_size %d must be a power of two, num_pages and max_blocks_per_seq positive",
                         op, page_size);
    if (v_head_stride < head_dim || v_tok_stride < (int64_t)num_heads_kv * v_head_stride)
        return set_error(EXL3R_EINVAL, "%s: v strides (%lld, %lld) overlap heads", op, (long long)v_tok_stride,
                         (long long)v_head_stride);
    if (num_pages > ((int64_t)1 << 62) / ((int64_t)page_size * num_heads_kv * (head_dim > 0 ? head_dim : 1)))
        return set_error(EXL3R_EINVAL, "%s: cache too large", op);
    if (bsz > 0 && seq_len > 0 && (!k || !v || !k_cache || !v_cache || !block_table || !cache_seqlens))
        return set_error(EXL3R_EINVAL, "%s: k, v, k_cache, v_cache, block_table and cache_seqlens must be non-null", op);
    const int rc = rope_prepare(op, a, q, out_q, q_tok_stride, q_head_stride, num_heads_q, k, out_k, true, k_tok_stride,
                                k_head_stride, num_heads_kv, dtype, bsz, seq_len, head_dim, inv_freq, rotary_dim, position,
                                positions, position_ids, q_norm, k_norm, norm_dtype, norm_eps, norm_constant_bias,
                                rope_mode, attn_factor);
    if (rc || a.tokens == 0) return rc;
    a.v = v; a.v_ts = v_tok_stride; a.v_hs = v_head_stride; a.hv = num_heads_kv;
    a.kc = k_cache; a.vc = v_cache;
    int lg = 0;
    while ((1 << lg) < page_size) ++lg;
    a.page_log2 = lg;
    a.pages = num_pages; a.max_blocks = max_blocks_per_seq;
    a.block_table = block_table; a.cache_seqlens = cache_seqlens; a.err = err_flag;
    return EXL3R_OK;
}

extern "C" int exl3r_rope_paged_kv(const void* q, void* out_q, int64_t q_tok_stride, int64_t q_head_stride,
                                   int num_heads_q, const void* k, void* out_k, int64_t k_tok_stride,
                                   int64_t k_head_stride, const void* v, int64_t v_tok_stride, int64_t v_head_stride,
                                   int num_heads_kv, int dtype, int64_t bsz, int64_t seq_len, int head_dim,
                                   const float* inv_freq, int rotary_dim,
                                   int32_t position, const int32_t* positions, const int32_t* position_ids,
                                   const void* q_norm, const void* k_norm, int norm_dtype,
                                   float norm_eps, float norm_constant_bias, int rope_mode, float attn_factor,
                                   void* k_cache, void* v_cache, int page_size, int64_t num_pages,
                                   const int32_t* block_table, int64_t max_blocks_per_seq,
                                   const int32_t* cache_seqlens, int32_t* err_flag, const void* cs_table,
                                   void* stream)
{
    begin_call();
    const char* op = "exl3r_rope_paged_kv";
    RopeArgs a;
    int rc = paged_prepare(op, a, q, out_q, q_tok_stride, q_head_stride, num_heads_q, k, out_k, k_tok_stride,
                           k_head_stride, v, v_tok_stride, v_head_stride, num_heads_kv, dtype, bsz, seq_len, head_dim,
                           rotation_source(inv_freq, cs_table), rotary_dim, position, positions, position_ids, q_norm,
                           k_norm, norm_dtype, norm_eps, norm_constant_bias, rope_mode, attn_factor, k_cache, v_cache,
                           page_size, num_pages, block_table, max_blocks_per_seq, cache_seqlens, err_flag);
    if (rc || a.tokens == 0) return rc;
    if ((rc = use_cs_table(op, a, cs_table))) return rc;
    return rope_dispatch(op, a, dtype, rope_mode, stream);
}

extern "C" int exl3r_rope_table(const void* q, void* out_q, int64_t q_tok_stride, int64_t q_head_stride, int num_heads_q,
                                const void* k, void* out_k, int64_t k_tok_stride, int64_t k_head_stride, int num_heads_k,
                                int dtype, int64_t bsz, int64_t seq_len, int head_dim,
                                const float* angle_table, int64_t table_rows, int64_t table_batch_stride, int rotary_dim,
                                int32_t position, const int32_t* positions, const int32_t* position_ids,
                                const void* q_norm, const void* k_norm, int norm_dtype,
                                float norm_eps, float norm_constant_bias, int rope_mode, float attn_factor,
                                int32_t* err_flag, void* stream)
{
    begin_call();
    const char* op = "exl3r_rope_table";
    if (table_rows <= 0 || table_batch_stride < 0)
        return set_error(EXL3R_EINVAL, "%s: table_rows must be positive and table_batch_stride non-negative", op);
    RopeArgs a;
    const int rc = rope_prepare(op, a, q, out_q, q_tok_stride, q_head_stride, num_heads_q, k, out_k, false, k_tok_stride,
                                k_head_stride, num_heads_k, dtype, bsz, seq_len, head_dim, angle_table, rotary_dim,
                                position, positions, position_ids, q_norm, k_norm, norm_dtype, norm_eps,
                                norm_constant_bias, rope_mode, attn_factor);
    if (rc || a.tokens == 0) return rc;
    a.table = angle_table;
    a.table_rows = table_rows;
    a.table_bstride = table_batch_stride;
    a.err = err_flag;
    return rope_dispatch(op, a, dtype, rope_mode, stream);
}

extern "C" int exl3r_had_r_128(const void* x, int dtype, int64_t ldx, void* out, int64_t ldo, int64_t rows,
                               int64_t cols, const void* pre_scale, const void* post_scale, float scale, void* stream);

// exl3r_rope with the q / k projections' output rotation first (Linear::forward's
// had_r_128(y, y, None, svh), src/modules.rs:231, then RoPE::apply on y).  Prefill-sized NeoX launches
// of f16 heads of 128 run it inside the wave-per-token kernel; anything else runs the rotations into
// out_q / out_k and exl3r_rope in place there.
extern "C" int exl3r_rope_had(const void* q, void* out_q, int64_t q_tok_stride, int num_heads_q,
                              const void* k, void* out_k, int64_t k_tok_stride, int num_heads_k,
                              int dtype, int64_t bsz, int64_t seq_len, int head_dim,
                              const float* inv_freq, int rotary_dim,
                              int32_t position, const int32_t* positions, const int32_t* position_ids,
                              const void* q_norm, const void* k_norm, int norm_dtype,
                              float norm_eps, float norm_constant_bias, int rope_mode, float attn_factor,
                              const void* q_post_scale, const void* k_post_scale, const void* cs_table, void* stream)
{
    begin_call();
    const char* op = "exl3r_rope_had";
    const bool exact = (rope_mode & EXL3R_HAD_EXACT) != 0;
    rope_mode &= ~EXL3R_HAD_EXACT;
    if (dtype != EXL3R_F16) return set_error(EXL3R_EDTYPE, "%s: the rotated projection outputs are f16", op);
    if (head_dim <= 0 || ((int64_t)num_heads_q * head_dim) % 128 || (k && ((int64_t)num_heads_k * head_dim) % 128))
        return set_error(EXL3R_EINVAL, "%s: heads * head_dim must be a multiple of 128", op);
    if (!k && (out_k || k_post_scale)) return set_error(EXL3R_EINVAL, "%s: out_k / k_post_scale without k", op);
    RopeArgs a;
    int rc = rope_prepare(op, a, q, out_q, q_tok_stride, head_dim, num_heads_q, k, out_k, false, k_tok_stride, head_dim,
                          num_heads_k, dtype, bsz, seq_len, head_dim, rotation_source(inv_freq, cs_table), rotary_dim,
                          position, positions, position_ids, q_norm, k_norm, norm_dtype, norm_eps, norm_constant_bias,
                          rope_mode, attn_factor);
    if (rc || a.tokens == 0) return rc;
    if ((rc = use_cs_table(op, a, cs_table))) return rc;
    a.q_post = q_post_scale;
    a.k_post = k_post_scale;
    if (rope_vec_ok(a, rope_mode) && rope_nx_ok(a, rope_mode, true))
    {
        hipStream_t s = (hipStream_t)stream;
        const int norm = rope_norm_kind(a, dtype);
        if (norm == NORM_NONE) launch_had_nx<NORM_NONE>(a, rope_mode, exact, s);
        else if (norm == NORM_HALF) launch_had_nx<NORM_HALF>(a, rope_mode, exact, s);
        else launch_had_nx<NORM_F32>(a, rope_mode, exact, s);
        return launch_status(op);
    }
    const bool fused = head_dim == 128 && rope_mode == EXL3R_ROPE_NEOX && rope_vec_ok(a, rope_mode) &&
                       rope_tok_launch(a) && (!q_post_scale || aligned16(q_post_scale)) &&
                       (!k_post_scale || aligned16(k_post_scale));
    if (fused)
    {
        hipStream_t s = (hipStream_t)stream;
        const int norm = rope_norm_kind(a, dtype);
        if (norm == NORM_NONE) launch_had_tok<NORM_NONE>(a, s);
        else if (norm == NORM_HALF) launch_had_tok<NORM_HALF>(a, s);
        else launch_had_tok<NORM_F32>(a, s);
        return launch_status(op);
    }
    const int64_t tokens = a.tokens;
    rc = exl3r_had_r_128(q, EXL3R_F16, q_tok_stride, out_q, q_tok_stride, tokens, (int64_t)num_heads_q * head_dim,
                         nullptr, q_post_scale, 1.0f, stream);
    if (rc == EXL3R_OK && k)
        rc = exl3r_had_r_128(k, EXL3R_F16, k_tok_stride, out_k, k_tok_stride, tokens, (int64_t)num_heads_k * head_dim,
                             nullptr, k_post_scale, 1.0f, stream);
    if (rc != EXL3R_OK) return rc;
    if (cs_table)
        return exl3r_rope_cs(out_q, out_q, q_tok_stride, head_dim, num_heads_q, k ? out_k : nullptr, k ? out_k : nullptr,
                             k_tok_stride, head_dim, num_heads_k, dtype, bsz, seq_len, head_dim, cs_table, rotary_dim,
                             q_norm, k_norm, norm_dtype, norm_eps, norm_constant_bias, rope_mode, stream);
    return exl3r_rope(out_q, out_q, q_tok_stride, head_dim, num_heads_q, k ? out_k : nullptr, k ? out_k : nullptr,
                      k_tok_stride, head_dim, num_heads_k, dtype, bsz, seq_len, head_dim, inv_freq, rotary_dim, position,
                      positions, position_ids, q_norm, k_norm, norm_dtype, norm_eps, norm_constant_bias, rope_mode,
                      attn_factor, stream);
}

// exl3r_rope_paged_kv preceded by the q / k / v projections' output rotation (Linear::forward's
// had_r_128(y, y, None, svh), src/modules.rs:231, then RoPE::apply and paged_kv_cache_update,
// src/modules.rs:669-704).  Prefill-sized NeoX launches of f16 heads of 128 run it inside the
// wave-per-token kernel; anything else rotates q into out_q, k into out_k (in place when out_k is
// null) and v in place, then runs exl3r_rope_paged_kv there.
extern "C" int exl3r_rope_paged_kv_had(const void* q, void* out_q, int64_t q_tok_stride, int num_heads_q,
                                       const void* k, void* out_k, int64_t k_tok_stride, const void* v,
                                       int64_t v_tok_stride, int num_heads_kv, int dtype, int64_t bsz,
                                       int64_t seq_len, int head_dim, const float* inv_freq, int rotary_dim,
                                       int32_t position, const int32_t* positions, const int32_t* position_ids,
                                       const void* q_norm, const void* k_norm, int norm_dtype,
                                       float norm_eps, float norm_constant_bias, int rope_mode, float attn_factor,
                                       void* k_cache, void* v_cache, int page_size, int64_t num_pages,
                                       const int32_t* block_table, int64_t max_blocks_per_seq,
                                       const int32_t* cache_seqlens, int32_t* err_flag,
                                       const void* q_post_scale, const void* k_post_scale, const void* v_post_scale,
                                       const void* cs_table, void* stream)
{
    begin_call();
    const char* op = "exl3r_rope_paged_kv_had";
    const bool exact = (rope_mode & EXL3R_HAD_EXACT) != 0;
    rope_mode &= ~EXL3R_HAD_EXACT;
    if (dtype != EXL3R_F16) return set_error(EXL3R_EDTYPE, "%s: the rotated projection outputs are f16", op);
    if (head_dim <= 0 || ((int64_t)num_heads_q * head_dim) % 128 || ((int64_t)num_heads_kv * head_dim) % 128)
        return set_error(EXL3R_EINVAL, "%s: heads * head_dim must be a multiple of 128", op);
    RopeArgs a;
    int rc = paged_prepare(op, a, q, out_q, q_tok_stride, head_dim, num_heads_q, k, out_k, k_tok_stride, head_dim, v,
                           v_tok_stride, head_dim, num_heads_kv, dtype, bsz, seq_len, head_dim,
                           rotation_source(inv_freq, cs_table), rotary_dim, position, positions, position_ids, q_norm,
                           k_norm, norm_dtype, norm_eps, norm_constant_bias, rope_mode, attn_factor, k_cache, v_cache,
                           page_size, num_pages, block_table, max_blocks_per_seq, cache_seqlens, err_flag);
    if (rc || a.tokens == 0) return rc;
    if ((rc = use_cs_table(op, a, cs_table))) return rc;
    a.q_post = q_post_scale;
    a.k_post = k_post_scale;
    a.v_post = v_post_scale;
    if (rope_vec_ok(a, rope_mode) && rope_nx_ok(a, rope_mode, true))
    {
        hipStream_t s = (hipStream_t)stream;
        const int norm = rope_norm_kind(a, dtype);
        if (norm == NORM_NONE) launch_had_nx<NORM_NONE>(a, rope_mode, exact, s);
        else if (norm == NORM_HALF) launch_had_nx<NORM_HALF>(a, rope_mode, exact, s);
        else launch_had_nx<NORM_F32>(a, rope_mode, exact, s);
        return launch_status(op);
    }
    auto a16 = [](const void* p) { return p == nullptr || aligned16(p); };
    const bool fused = head_dim == 128 && rope_mode == EXL3R_ROPE_NEOX && rope_vec_ok(a, rope_mode) &&
                       rope_tok_launch(a) && a16(q_post_scale) && a16(k_post_scale) && a16(v_post_scale);
    if (fused)
    {
        hipStream_t s = (hipStream_t)stream;
        const int norm = rope_norm_kind(a, dtype);
        if (norm == NORM_NONE) launch_had_tok<NORM_NONE>(a, s);
        else if (norm == NORM_HALF) launch_had_tok<NORM_HALF>(a, s);
        else launch_had_tok<NORM_F32>(a, s);
        return launch_status(op);
    }
    const int64_t tokens = a.tokens;
    void* kr = out_k ? out_k : const_cast<void*>(k);
    rc = exl3r_had_r_128(q, EXL3R_F16, q_tok_stride, out_q, q_tok_stride, tokens, (int64_t)num_heads_q * head_dim,
                         nullptr, q_post_scale, 1.0f, stream);
    if (rc == EXL3R_OK)
        rc = exl3r_had_r_128(k, EXL3R_F16, k_tok_stride, kr, k_tok_stride, tokens, (int64_t)num_heads_kv * head_dim,
                             nullptr, k_post_scale, 1.0f, stream);
    if (rc == EXL3R_OK)
        rc = exl3r_had_r_128(v, EXL3R_F16, v_tok_stride, const_cast<void*>(v), v_tok_stride, tokens,
                             (int64_t)num_heads_kv * head_dim, nullptr, v_post_scale, 1.0f, stream);
    if (rc != EXL3R_OK) return rc;
    return exl3r_rope_paged_kv(out_q, out_q, q_tok_stride, head_dim, num_heads_q, kr, out_k, k_tok_stride, head_dim, v,
                               v_tok_stride, head_dim, num_heads_kv, dtype, bsz, seq_len, head_dim, inv_freq,
                               rotary_dim, position, positions, position_ids, q_norm, k_norm, norm_dtype, norm_eps,
                               norm_constant_bias, rope_mode, attn_factor, k_cache, v_cache, page_size, num_pages,
                               block_table, max_blocks_per_seq, cache_seqlens, err_flag, cs_table, stream);
}

// {cos, sin} * attn_factor of every token's rotary frequencies into cs_table [bsz * seq_len, R / 2]
// (float2), for exl3r_rope_cs: the positions of a forward pass are the same in every layer, so the
// table is built once and every layer's RoPE reads it.  Positions as exl3r_rope.
extern "C" int exl3r_rope_cs_table(int64_t bsz, int64_t seq_len, const float* inv_freq, int rotary_dim,
                                   int32_t position, const int32_t* positions, const int32_t* position_ids,
                                   float attn_factor, void* cs_table, void* stream)
{
    begin_call();
    const char* op = "exl3r_rope_cs_table";
    if (bsz < 0 || seq_len < 0 || rotary_dim < 2 || rotary_dim % 2)
        return set_error(EXL3R_EINVAL, "%s: invalid shape bsz=%lld seq_len=%lld rotary_dim=%d", op, (long long)bsz,
                         (long long)seq_len, rotary_dim);
    if (positions && position_ids) return set_error(EXL3R_EINVAL, "%s: at most one of positions / position_ids", op);
    const int64_t tokens = bsz * seq_len;
    if (tokens == 0) return EXL3R_OK;
    if (!inv_freq || !cs_table) return set_error(EXL3R_EINVAL, "%s: inv_freq and cs_table must be non-null", op);
    if ((uintptr_t)cs_table % 8) return set_error(EXL3R_EINVAL, "%s: cs_table must be 8-byte aligned", op);
    if (tokens > 0x7fffffff) return set_error(EXL3R_EINVAL, "%s: too many tokens", op);
    RopeArgs a{};
    a.R = rotary_dim; a.seq_len = seq_len; a.tokens = tokens; a.inv_freq = inv_freq; a.position = position;
    a.positions = positions; a.position_ids = position_ids; a.attn = attn_factor;
    const int64_t n = tokens * (rotary_dim / 2);
    const unsigned blocks = (unsigned)((n + 255) / 256 < kMaxGridX ? (n + 255) / 256 : kMaxGridX);
    launch(k_rope_cs_table, blocks, 256, 0, (hipStream_t)stream, a, (float2*)cs_table);
    return launch_status(op);
}

// exl3r_rope with the rotary pairs read from a table built by exl3r_rope_cs_table (same positions,
// inv_freq, rotary_dim and attn_factor): bit-identical to exl3r_rope, on the same kernels and shapes.
extern "C" int exl3r_rope_cs(const void* q, void* out_q, int64_t q_tok_stride, int64_t q_head_stride,
                             int num_heads_q, const void* k, void* out_k, int64_t k_tok_stride,
                             int64_t k_head_stride, int num_heads_k, int dtype, int64_t bsz, int64_t seq_len,
                             int head_dim, const void* cs_table, int rotary_dim, const void* q_norm,
                             const void* k_norm, int norm_dtype, float norm_eps, float norm_constant_bias,
                             int rope_mode, void* stream)
{
    begin_call();
    const char* op = "exl3r_rope_cs";
    if (!cs_table && bsz > 0 && seq_len > 0) return set_error(EXL3R_EINVAL, "%s: cs_table must be non-null", op);
    // rope_prepare checks the rotation source of exl3r_rope; the table of an empty call may be NULL.
    static const float kEmpty = 0.0f;
    RopeArgs a;
    int rc = rope_prepare(op, a, q, out_q, q_tok_stride, q_head_stride, num_heads_q, k, out_k, false, k_tok_stride,
                          k_head_stride, num_heads_k, dtype, bsz, seq_len, head_dim,
                          cs_table ? (const float*)cs_table : &kEmpty, rotary_dim,
                          0, nullptr, nullptr, q_norm, k_norm, norm_dtype, norm_eps, norm_constant_bias, rope_mode, 1.0f);
    if (rc || a.tokens == 0) return rc;
    if ((uintptr_t)cs_table % 8) return set_error(EXL3R_EINVAL, "%s: cs_table must be 8-byte aligned", op);
    a.inv_freq = nullptr;
    a.cst = (const float2*)cs_table;
    rc = rope_dispatch(op, a, dtype, rope_mode, stream);
    return rc;
}

// exl3r_deinterleave_qg followed by exl3r_rope on q (and k), in one pass: the q half of each head's
// interleaved [q | g] pair is read straight from qg and written roped (and normed) to a dense out_q;
// g stays in qg for exl3r_mul_sigmoid with a row stride of 2 * head_dim.
extern "C" int exl3r_rope_qg(const void* qg, int64_t qg_tok_stride, void* out_q, int num_heads_q, const void* k,
                             void* out_k, int64_t k_tok_stride, int64_t k_head_stride, int num_heads_k, int dtype,
                             int64_t bsz, int64_t seq_len, int head_dim, const float* inv_freq, int rotary_dim,
                             int32_t position, const int32_t* positions, const int32_t* position_ids,
                             const void* q_norm, const void* k_norm, int norm_dtype, float norm_eps,
                             float norm_constant_bias, int rope_mode, float attn_factor, void* stream)
{
    begin_call();
    const char* op = "exl3r_rope_qg";
    if (head_dim <= 0 || head_dim > 4096)
        return set_error(EXL3R_EINVAL, "%s: head_dim %d must be in [2, 4096]", op, head_dim);
    RopeArgs a;
    int rc = rope_prepare(op, a, qg, out_q, qg_tok_stride, 2 * (int64_t)head_dim, num_heads_q, k, out_k, false,
                          k_tok_stride, k_head_stride, num_heads_k, dtype, bsz, seq_len, head_dim, inv_freq, rotary_dim,
                          position, positions, position_ids, q_norm, k_norm, norm_dtype, norm_eps, norm_constant_bias,
                          rope_mode, attn_factor);
    if (rc || a.tokens == 0) return rc;
    a.oq_hs = head_dim;
    a.oq_ts = (int64_t)num_heads_q * head_dim;
    // out_q is written while qg is read by other workgroups: the two must not overlap.
    const int es = dtype_bytes(dtype);
    const char* q0 = (const char*)qg;
    const char* q1 = q0 + ((a.tokens - 1) * qg_tok_stride + 2 * (int64_t)num_heads_q * head_dim) * es;
    const char* o0 = (const char*)out_q;
    const char* o1 = o0 + a.tokens * a.oq_ts * es;
    if (o0 < q1 && q0 < o1) return set_error(EXL3R_EINVAL, "%s: out_q overlaps qg", op);
    return rope_dispatch(op, a, dtype, rope_mode, stream);
}

// The descriptor form of every RoPE entry point above: checks that one variant is named, then calls
// its entry point, whose checks, results and errors it has.
extern "C" int exl3r_rope_run(const exl3r_rope_desc* d, void* stream)
{
    begin_call();
    const char* op = "exl3r_rope_run";
    if (!d) return set_error(EXL3R_EINVAL, "%s: descriptor must be non-null", op);
    if (d->struct_size < (int32_t)sizeof(exl3r_rope_desc))
        return set_error(EXL3R_EINVAL, "%s: struct_size %d < sizeof(exl3r_rope_desc) %d", op, d->struct_size,
                         (int)sizeof(exl3r_rope_desc));
    // A zero-initialised descriptor leaves attn_factor 0, which would scale every {cos, sin} pair to
    // zero and return zeroed q / k as a success: refused, 1.0 being the unscaled rotation.
    if (d->attn_factor == 0.0f || d->attn_factor != d->attn_factor)
        return set_error(EXL3R_EINVAL, "%s: attn_factor %g (1.0 for no scaling; a zero-initialised descriptor must set it)",
                         op, (double)d->attn_factor);
    const int sources = (d->inv_freq != nullptr) + (d->angle_table != nullptr) + (d->cs_table != nullptr);
    const bool cs_with_freq = d->cs_table && d->inv_freq && !d->angle_table;   // rotate / k_cache forms
    if (sources == 0) return set_error(EXL3R_EINVAL, "%s: no rotation source (inv_freq, angle_table or cs_table)", op);
    if (sources > 1 && !(cs_with_freq && (d->rotate || d->k_cache)))
        return set_error(EXL3R_EINVAL, "%s: more than one rotation source", op);
    const int64_t oq_ts = d->out_q_tok_stride ? d->out_q_tok_stride : d->q_tok_stride;
    const int64_t oq_hs = d->out_q_head_stride ? d->out_q_head_stride : d->q_head_stride;
    const bool own_layout = oq_ts != d->q_tok_stride || oq_hs != d->q_head_stride;
    const bool post = d->q_post_scale || d->k_post_scale || d->v_post_scale;
    if (!d->rotate && post) return set_error(EXL3R_EINVAL, "%s: post-scales given without rotate", op);
    if (!d->k_cache && (d->v || d->v_cache || d->block_table || d->cache_seqlens))
        return set_error(EXL3R_EINVAL, "%s: v / v_cache / block_table / cache_seqlens given without k_cache", op);
    if ((d->rotate || d->k_cache) && d->angle_table)
        return set_error(EXL3R_EINVAL, "%s: the rotating and paged forms take inv_freq or cs_table, not an angle table", op);
    if (own_layout && (d->rotate || d->k_cache || d->angle_table || d->cs_table))
        return set_error(EXL3R_EINVAL, "%s: an out_q layout of its own is the q | g split only (inv_freq, no cache, no rotation)", op);
    const int64_t hd = d->head_dim;
    if (d->rotate != 0 && d->rotate != 1 && d->rotate != (1 | EXL3R_HAD_EXACT))
        return set_error(EXL3R_EINVAL, "%s: rotate takes 0, 1 or 1 | EXL3R_HAD_EXACT", op);
    if (d->rotate)
    {
        // The rotating forms take packed heads (head stride = head_dim); EXL3R_HAD_EXACT goes to their
        // rope_mode.
        const int mode = d->rope_mode | (d->rotate & EXL3R_HAD_EXACT);
        if (d->q_head_stride != hd || (d->k && d->k_head_stride != hd) || (d->v && d->v_head_stride != hd))
            return set_error(EXL3R_EINVAL, "%s: rotate takes packed heads (head strides equal to head_dim)", op);
        if (d->k_cache)
            return exl3r_rope_paged_kv_had(d->q, d->out_q, d->q_tok_stride, d->num_heads_q, d->k, d->out_k, d->k_tok_stride,
                                           d->v, d->v_tok_stride, d->num_heads_k, d->dtype, d->bsz, d->seq_len,
                                           d->head_dim, d->inv_freq, d->rotary_dim, d->position, d->positions,
                                           d->position_ids, d->q_norm, d->k_norm, d->norm_dtype, d->norm_eps,
                                           d->norm_constant_bias, mode, d->attn_factor, d->k_cache, d->v_cache,
                                           d->page_size, d->num_pages, d->block_table, d->max_blocks_per_seq,
                                           d->cache_seqlens, d->err_flag, d->q_post_scale, d->k_post_scale,
                                           d->v_post_scale, d->cs_table, stream);
        return exl3r_rope_had(d->q, d->out_q, d->q_tok_stride, d->num_heads_q, d->k, d->out_k, d->k_tok_stride,
                              d->num_heads_k, d->dtype, d->bsz, d->seq_len, d->head_dim, d->inv_freq, d->rotary_dim,
                              d->position, d->positions, d->position_ids, d->q_norm, d->k_norm, d->norm_dtype,
                              d->norm_eps, d->norm_constant_bias, mode, d->attn_factor, d->q_post_scale,
                              d->k_post_scale, d->cs_table, stream);
    }
    if (d->k_cache)
        return exl3r_rope_paged_kv(d->q, d->out_q, d->q_tok_stride, d->q_head_stride, d->num_heads_q, d->k, d->out_k,
                                   d->k_tok_stride, d->k_head_stride, d->v, d->v_tok_stride, d->v_head_stride,
                                   d->num_heads_k, d->dtype, d->bsz, d->seq_len, d->head_dim, d->inv_freq,
                                   d->rotary_dim, d->position, d->positions, d->position_ids, d->q_norm, d->k_norm,
                                   d->norm_dtype, d->norm_eps, d->norm_constant_bias, d->rope_mode, d->attn_factor,
                                   d->k_cache, d->v_cache, d->page_size, d->num_pages, d->block_table,
                                   d->max_blocks_per_seq, d->cache_seqlens, d->err_flag, d->cs_table, stream);
    if (d->angle_table)
        return exl3r_rope_table(d->q, d->out_q, d->q_tok_stride, d->q_head_stride, d->num_heads_q, d->k, d->out_k,
                                d->k_tok_stride, d->k_head_stride, d->num_heads_k, d->dtype, d->bsz, d->seq_len,
                                d->head_dim, d->angle_table, d->table_rows, d->table_batch_stride, d->rotary_dim,
                                d->position, d->positions, d->position_ids, d->q_norm, d->k_norm, d->norm_dtype,
                                d->norm_eps, d->norm_constant_bias, d->rope_mode, d->attn_factor, d->err_flag, stream);
    if (own_layout)
    {
        if (d->q_head_stride != 2 * hd || oq_hs != hd || oq_ts != (int64_t)d->num_heads_q * hd)
            return set_error(EXL3R_EINVAL, "%s: an out_q layout of its own is the q | g split: q head stride 2 * head_dim "
                             "and a dense out_q", op);
        return exl3r_rope_qg(d->q, d->q_tok_stride, d->out_q, d->num_heads_q, d->k, d->out_k, d->k_tok_stride,
                             d->k_head_stride, d->num_heads_k, d->dtype, d->bsz, d->seq_len, d->head_dim, d->inv_freq,
                             d->rotary_dim, d->position, d->positions, d->position_ids, d->q_norm, d->k_norm,
                             d->norm_dtype, d->norm_eps, d->norm_constant_bias, d->rope_mode, d->attn_factor, stream);
    }
    if (d->cs_table)
        return exl3r_rope_cs(d->q, d->out_q, d->q_tok_stride, d->q_head_stride, d->num_heads_q, d->k, d->out_k,
                             d->k_tok_stride, d->k_head_stride, d->num_heads_k, d->dtype, d->bsz, d->seq_len, d->head_dim,
                             d->cs_table, d->rotary_dim, d->q_norm, d->k_norm, d->norm_dtype, d->norm_eps,
                             d->norm_constant_bias, d->rope_mode, stream);
    return exl3r_rope(d->q, d->out_q, d->q_tok_stride, d->q_head_stride, d->num_heads_q, d->k, d->out_k, d->k_tok_stride,
                      d->k_head_stride, d->num_heads_k, d->dtype, d->bsz, d->seq_len, d->head_dim, d->inv_freq,
                      d->rotary_dim, d->position, d->positions, d->position_ids, d->q_norm, d->k_norm, d->norm_dtype,
                      d->norm_eps, d->norm_constant_bias, d->rope_mode, d->attn_factor, stream);
}
