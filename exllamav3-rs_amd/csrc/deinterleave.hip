// C ABI: exl3r_deinterleave_qg (replaces exl3_shim_deinterleave_qg, reference csrc/exl3_shim.cpp:168-171 ->
// deinterleave_qg, kernels/activation.cu:721-779; called by the gated-attention q projection,
// src/modules.rs:637-646, 800-808): rows of per-head interleaved [heads, q | g] (2 * head_dim each) are
// split into q [rows, heads, head_dim] and g [rows, heads * head_dim].  A bit copy.
//
// Layout: grid.y walks rows, grid.x the 16-byte chunks of one row's q and g halves; each lane moves
// one chunk of q and the matching chunk of g (non-temporal: every byte is touched once).
#include "abi.hpp"
#include "common.cuh"

namespace exl3r {

struct QgArgs
{
    const char* qg;
    char* q;
    char* g;
    int64_t ldqg, ldq, ldg;   // row strides, bytes
    int64_t rows;
    int heads;
    int hb;                   // bytes per head half (head_dim * element size)
};

__global__ __launch_bounds__(256) void k_deinterleave_qg(QgArgs a)
{
    const int hc = a.hb >> 4;                         // 16-byte chunks per head half
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= a.heads * hc) return;
    const int h = j / hc;
    const int c = j - h * hc;
    for (int64_t r = blockIdx.y; r < a.rows; r += gridDim.y)
    {
        const u32x4* src = (const u32x4*)(a.qg + r * a.ldqg + (int64_t)h * 2 * a.hb) + c;
        const u32x4 qv = __builtin_nontemporal_load(src);
        const u32x4 gv = __builtin_nontemporal_load(src + hc);
        __builtin_nontemporal_store(qv, (u32x4*)(a.q + r * a.ldq + (int64_t)h * a.hb) + c);
        __builtin_nontemporal_store(gv, (u32x4*)(a.g + r * a.ldg + (int64_t)h * a.hb) + c);
    }
}

// Any alignment: one 2-byte (or 4-byte) element per lane.
__global__ __launch_bounds__(256) void k_deinterleave_qg_generic(QgArgs a, int es)
{
    const int hd = a.hb / es;
    const int64_t n = a.rows * a.heads * hd;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    {
        const int64_t rh = i / hd;
        const int d = (int)(i - rh * hd);
        const int64_t r = rh / a.heads;
        const int h = (int)(rh - r * a.heads);
        const char* src = a.qg + r * a.ldqg + ((int64_t)h * 2 * hd + d) * es;
        char* dq = a.q + r * a.ldq + ((int64_t)h * hd + d) * es;
        char* dg = a.g + r * a.ldg + ((int64_t)h * hd + d) * es;
        if (es == 2)
        {
            *(uint16_t*)dq = *(const uint16_t*)src;
            *(uint16_t*)dg = *(const uint16_t*)(src + a.hb);
        }
        else
        {
            *(uint32_t*)dq = *(const uint32_t*)src;
            *(uint32_t*)dg = *(const uint32_t*)(src + a.hb);
        }
    }
}

}  // namespace exl3r

using namespace exl3r;

extern "C" int exl3r_deinterleave_qg(const void* qg, int64_t ld_qg, void* q, int64_t ld_q, void* g, int64_t ld_g,
                                     int dtype, int64_t rows, int heads, int head_dim, void* stream)
{
    begin_call();
    const char* op = "exl3r_deinterleave_qg";
    if (!is_float_dtype(dtype)) return set_error(EXL3R_EDTYPE, "%s: unsupported dtype %s", op, dtype_name(dtype));
    if (rows < 0 || heads <= 0 || head_dim <= 0 || (int64_t)heads * head_dim > ((int64_t)1 << 28))
        return set_error(EXL3R_EINVAL, "%s: invalid shape rows=%lld heads=%d head_dim=%d", op, (long long)rows, heads, head_dim);
    const int64_t width = (int64_t)heads * head_dim;
    if (rows > 1 && (ld_qg < 2 * width || ld_q < width || ld_g < width))
        return set_error(EXL3R_EINVAL, "%s: row strides must cover the rows", op);
    if (rows == 0) return EXL3R_OK;
    if (!qg || !q || !g) return set_error(EXL3R_EINVAL, "%s: qg, q and g must be non-null", op);
    if (q == g || q == qg || g == qg) return set_error(EXL3R_EINVAL, "%s: q, g and qg must not alias", op);

    const int es = dtype_bytes(dtype);
    QgArgs a{ (const char*)qg, (char*)q, (char*)g, ld_qg * es, ld_q * es, ld_g * es, rows, heads, head_dim * es };
    hipStream_t s = (hipStream_t)stream;
    const bool vec = a.hb % 16 == 0 && aligned16(qg) && aligned16(q) && aligned16(g) &&
                     (rows == 1 || (a.ldqg % 16 == 0 && a.ldq % 16 == 0 && a.ldg % 16 == 0));
    if (vec)
    {
        const int chunks = heads * (a.hb >> 4);
        // one-wave workgroups (Qwen3.5 [4096, 32, 2 x 128] f16, same process, both orders: 23.7-24.0 against
        // 24.9-25.0 us with 256 lanes)
        constexpr int kThreads = 64;
        const dim3 grid((unsigned)((chunks + kThreads - 1) / kThreads), (unsigned)(rows < 65535 ? rows : 65535));
        launch(k_deinterleave_qg, grid, kThreads, 0, s, a);
    }
    else
    {
        const int64_t n = rows * width;
        launch(k_deinterleave_qg_generic, (unsigned)((n + 255) / 256 < kMaxGridX ? (n + 255) / 256 : kMaxGridX), 256, 0, s, a, es);
    }
    return launch_status(op);
}
