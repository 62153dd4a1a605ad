// Token-embedding gather for gfx950: exl3r_embedding (replaces Embedding::forward's tch
// index_select + to_kind(Float), reference src/modules.rs:430-436) and exl3r_embedding_rms_norm
// (the gather fused with the RMSNorm that follows it, as the MTP head applies
// pre_fc_norm_embedding to embed(t), reference src/mtp.rs:189-190).
//
// The gather is a pure copy: 8-element chunks per lane, one workgroup per token row, copied
// bit-for-bit when out has the table's dtype and upcast exactly to F32 otherwise.  With an f32 side
// and rows of whole 512-element spans the chunks are split (two quads 256 apart), so that every
// wave-wide f32 access is one contiguous 1 KB (MI355X: bf16 table -> f32 rows at [16384, 5120] Zipf,
// see the launch).  Ids outside [0, vocab) produce a zero row and set the caller's device error flag.
#include "rms_norm_kernel.cuh"
#include "rms_norm_launch.hpp"

namespace exl3r {

struct EmbArgs
{
    const void* table;
    int64_t ldt, vocab;
    const void* ids;
    int idt;
    void* out;
    int64_t ldo;
    int64_t n;
    int hidden;
    int32_t* err;
};

template <class TT, class OT, int UNROLL, bool SPLIT = false>
__global__ __launch_bounds__(1024) void k_embedding(EmbArgs a)
{
    const int nc = a.hidden >> 3;
    const int nt = blockDim.x;
    for (int64_t row = blockIdx.x; row < a.n; row += gridDim.x)
    {
        int64_t id = load_id(a.ids, a.idt, row);
        const bool valid = id >= 0 && id < a.vocab;
        if (!valid && threadIdx.x == 0 && a.err) atomicOr(a.err, 1);
        const char* src = (const char*)a.table + (valid ? id : 0) * a.ldt * TT::bytes;
        char* dst = (char*)a.out + row * a.ldo * OT::bytes;
        for (int base = threadIdx.x; base < nc; base += nt * UNROLL)
        {
            typename TT::Vec v[UNROLL];
            #pragma unroll
            for (int u = 0; u < UNROLL; ++u)
            {
                const int c = base + u * nt;
                if (c < nc && valid)
                {
                    if constexpr (SPLIT) v[u] = load8_split<TT>(src, chunk_elem<true>(c));
                    else v[u] = load8<TT>(src, (int64_t)c * 8);
                }
            }
            #pragma unroll
            for (int u = 0; u < UNROLL; ++u)
            {
                const int c = base + u * nt;
                if (c < nc)
                {
                    const int64_t e = chunk_elem<SPLIT>(c);
                    auto put = [&](const typename OT::Vec& o) {
                        if constexpr (SPLIT) store8_split<OT>(dst, e, o);
                        else store8<OT>(dst, e, o);
                    };
                    if constexpr (TT::code == OT::code)
                    {
                        if (!valid)
                        {
                            const float z[8] = {};
                            v[u] = pack8<TT>(z);
                        }
                        put(v[u]);
                    }
                    else
                    {
                        float f[8];
                        if (valid) unpack8<TT>(v[u], f);
                        else
                        {
                            #pragma unroll
                            for (int j = 0; j < 8; ++j) f[j] = 0.0f;
                        }
                        put(pack8<OT>(f));
                    }
                }
            }
        }
    }
}

// Generic fallback: element-granular copy (any hidden size / alignment).
__global__ __launch_bounds__(256) void k_embedding_generic(EmbArgs a, int tt, int ot)
{
    for (int64_t row = blockIdx.x; row < a.n; row += gridDim.x)
    {
        int64_t id = load_id(a.ids, a.idt, row);
        const bool valid = id >= 0 && id < a.vocab;
        if (!valid && threadIdx.x == 0 && a.err) atomicOr(a.err, 1);
        for (int j = threadIdx.x; j < a.hidden; j += blockDim.x)
        {
            if (tt == ot && ot != DT_F32)
                ((uint16_t*)a.out)[row * a.ldo + j] = valid ? ((const uint16_t*)a.table)[id * a.ldt + j] : 0;
            else
                store1(a.out, ot, row * a.ldo + j, valid ? load1(a.table, tt, id * a.ldt + j) : 0.0f);
        }
    }
}

static bool exact_conversion(int from, int to) { return from == to || to == EXL3R_F32; }

static int check_gather(const char* op, const void* table, int tt, int64_t vocab, int64_t hidden, int64_t ldt,
                        const void* ids, int idt, int64_t n)
{
    if (!table || (n > 0 && !ids)) return set_error(EXL3R_EINVAL, "%s: table and ids must be non-null", op);
    if (vocab <= 0 || hidden <= 0 || hidden > (int64_t)1 << 30 || n < 0 || ldt < hidden)
        return set_error(EXL3R_EINVAL, "%s: invalid shape vocab=%lld hidden=%lld n=%lld ldt=%lld", op, (long long)vocab,
                         (long long)hidden, (long long)n, (long long)ldt);
    if (!is_float_dtype(tt)) return set_error(EXL3R_EDTYPE, "%s: unsupported table dtype %s", op, dtype_name(tt));
    if (idt != EXL3R_I32 && idt != EXL3R_I64) return set_error(EXL3R_EDTYPE, "%s: ids must be i32 or i64", op);
    return EXL3R_OK;
}

}  // namespace exl3r

using namespace exl3r;

extern "C" int exl3r_embedding(const void* table, int tt, int64_t vocab, int64_t hidden, int64_t ldt,
                               const void* ids, int idt, int64_t n, void* out, int ot, int64_t ldo,
                               int32_t* err_flag, void* stream)
{
    begin_call();
    const char* op = "exl3r_embedding";
    int rc = check_gather(op, table, tt, vocab, hidden, ldt, ids, idt, n);
    if (rc) return rc;
    if (n > 0 && !out) return set_error(EXL3R_EINVAL, "%s: out must be non-null", op);
    if (ldo < hidden) return set_error(EXL3R_EINVAL, "%s: out row stride %lld < hidden %lld", op, (long long)ldo, (long long)hidden);
    if (!is_float_dtype(ot) || !exact_conversion(tt, ot))
        return set_error(EXL3R_EDTYPE, "%s: out dtype %s is not an exact copy of table dtype %s", op, dtype_name(ot), dtype_name(tt));
    if (n == 0) return EXL3R_OK;

    EmbArgs a{ table, ldt, vocab, ids, idt, out, ldo, n, (int)hidden, err_flag };
    hipStream_t s = (hipStream_t)stream;
    const unsigned grid = (unsigned)(n < kMaxGridX ? n : kMaxGridX);
    const bool vec = hidden % 8 == 0 && aligned16(table) && aligned16(out) &&
                     (ldt * dtype_bytes(tt)) % 16 == 0 && (ldo * dtype_bytes(ot)) % 16 == 0;
    if (vec)
    {
        const int nc = (int)(hidden / 8);
        const Tuning& tu = tuning();
        int threads = (tu.embed_threads > 0 && tu.embed_threads % 64 == 0 && tu.embed_threads <= 1024) ? tu.embed_threads
                      : nc >= 1024 ? 256 : ((nc / 4 + 63) / 64) * 64;
        if (threads < 64) threads = 64;
        const bool split = nc % 64 == 0 && (tt == EXL3R_F32 || ot == EXL3R_F32) && tu.rms_split != -1;
        with_float_type(tt, [&](auto T) {
            with_float_type(ot, [&](auto O) {
                using TTy = decltype(T);
                using OTy = decltype(O);
                if constexpr (TTy::code == OTy::code || OTy::code == DT_F32)
                {
                    if (split) launch(k_embedding<TTy, OTy, 4, true>, grid, threads, 0, s, a);
                    else launch(k_embedding<TTy, OTy, 4>, grid, threads, 0, s, a);
                }
            });
        });
    }
    else
        launch(k_embedding_generic, grid, 256, 0, s, a, tt, ot);
    return launch_status(op);
}

extern "C" int exl3r_embedding_rms_norm(const void* table, int tt, int64_t vocab, int64_t hidden, int64_t ldt,
                                        const void* ids, int idt, int64_t n,
                                        void* h, int ht, int64_t ldh,
                                        const void* w, int wt, void* y, int yt, int64_t ldy,
                                        float eps, float constant_bias, float constant_scale,
                                        int32_t* err_flag, void* stream)
{
    begin_call();
    const char* op = "exl3r_embedding_rms_norm";
    int rc = check_gather(op, table, tt, vocab, hidden, ldt, ids, idt, n);
    if (rc) return rc;
    rc = check_rms_common(op, table, tt, ldt, w, wt, y, yt, ldy, n, hidden);
    if (rc) return rc;
    if (h && (ldh < hidden || !is_float_dtype(ht) || !exact_conversion(tt, ht)))
        return set_error(EXL3R_EINVAL, "%s: h must be an exact copy of the table dtype (or f32) with stride >= hidden", op);
    if (n > 0 && h && h == y) return set_error(EXL3R_EINVAL, "%s: h must not alias y", op);
    if (n == 0) return EXL3R_OK;

    RmsArgs a{};
    a.x = table; a.ldx = ldt; a.w = w; a.wt = wt; a.y = y; a.ldy = ldy; a.r = h; a.ldr = ldh;
    a.ids = ids; a.idt = idt; a.vocab = vocab; a.err = err_flag;
    a.rows = n; a.dim = (int)hidden; a.eps = eps; a.cb = constant_bias; a.cs = constant_scale;
    hipStream_t s = (hipStream_t)stream;

    if (rms_vec_ok(a, tt, yt, h ? ht : tt, h != nullptr, RMS_GATHER, 0))
    {
        with_float_type(tt, [&](auto T) {
            with_float_type(yt, [&](auto Y) {
                using TTy = decltype(T);
                using YTy = decltype(Y);
                if (!h) launch_rms_vec<TTy, YTy, TNone, RMS_GATHER>(a, s);
                else if (ht == tt) launch_rms_vec<TTy, YTy, TTy, RMS_GATHER>(a, s);
                else launch_rms_vec<TTy, YTy, TF32, RMS_GATHER>(a, s);
            });
        });
    }
    else
    {
        const unsigned grid = (unsigned)(n < kMaxGridX ? n : kMaxGridX);
        launch(k_rms_norm_generic<RMS_GATHER>, grid, 256, 0, s, a, tt, yt, h ? ht : tt);
    }
    return launch_status(op);
}
