// Host-side helpers shared by the C ABI entry points: thread-local error message, argument
// validation, kernel launches that report their own status.  Nothing here allocates or synchronises.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <tuple>
#include <type_traits>
#include <utility>

#include "../../include/exl3r/rowops.h"

namespace exl3r {

// Records a printf-style message for exl3r_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Launch status of the current entry point call, kept in this library's own thread-local slot.
// Launches go through hipLaunchKernel, whose return value is that launch's own status, so the
// thread's HIP last-error state is never read or cleared: an error that another caller (torch, the
// application) left pending stays where it was.
inline thread_local hipError_t t_launch_error = hipSuccess;

// Every entry point starts with begin_call(), before validating its arguments.
inline void begin_call() { t_launch_error = hipSuccess; }

// The first failed launch of this call, or EXL3R_OK; sets the message on failure.
int launch_status(const char* op);

// k<<<grid, block, shmem, stream>>>(args...) with the launch's own status: recorded for
// launch_status and returned (as an int hipError_t).  Each argument is converted to its kernel
// parameter's type.
template <class... P, class... A>
inline int launch(void (*k)(P...), dim3 grid, dim3 block, size_t shmem, hipStream_t stream, A&&... args)
{
    static_assert(sizeof...(P) == sizeof...(A), "one argument per kernel parameter");
    std::tuple<std::remove_cv_t<P>...> vals(std::forward<A>(args)...);
    void* argv[sizeof...(P) > 0 ? sizeof...(P) : 1] = {};
    std::apply([&](auto&... v) {
        int i = 0;
        ((argv[i++] = (void*)&v), ...);
    }, vals);
    const hipError_t e = hipLaunchKernel(reinterpret_cast<const void*>(k), grid, block, argv, shmem, stream);
    if (e != hipSuccess && t_launch_error == hipSuccess) t_launch_error = e;
    return (int)e;
}

inline bool is_float_dtype(int dt) { return dt == EXL3R_F32 || dt == EXL3R_F16 || dt == EXL3R_BF16; }
inline int dtype_bytes(int dt)
{
    switch (dt)
    {
        case EXL3R_F32: case EXL3R_I32: return 4;
        case EXL3R_F16: case EXL3R_BF16: return 2;
        case EXL3R_I64: return 8;
        default: return 0;
    }
}
inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
const char* dtype_name(int dt);

// Grid rows are walked with a stride loop beyond this many workgroups.
constexpr int64_t kMaxGridX = 1 << 20;

// Launch-shape overrides (0 = automatic).  The product library is built without EXL3R_TUNING: every
// field is then a compile-time zero and the shape rules below are fixed.  The sweep/test build
// (lib/libexl3rowops_tune.so, EXL3R_TUNING defined) exports exl3r_tune_* (csrc/tuning.h), which set
// them process-wide.
struct Tuning
{
    int rms_maxv = 0, rms_threads = 0;
    int rms_rows_rpl = 0;
    int rms_split = 0, rms_split_wm = 1;   // split chunks: -1 never, 0 auto, 1 always; weight mode (1 mid, 2 late)
    int rms_sum32 = 0;                     // plain / residual norms: 1 = fp32 row sum (0: fp64)
    int rms_wmode = 0;                     // streaming plain / residual norms: weight fetched 1 early, 2 mid, 3 late (0 auto)
    int rms_r_cached = 0;                  // Hadamard norms: 1 = cached residual stores
    int rms_pipe = 0;                      // streaming plain / residual norms: 1 = resident grid, as many
                                           // workgroups per CU as fit; n > 1: n - 1 per CU
    int act_unroll = 0, act_threads = 0, act_blocks_per_cu = 0;
    int rope_iters = 0;
    int rope_tok = 0;       // 0 auto, 1 never the wave-per-token kernel, 2 always (where it applies)
    int rope_hpl = 0;       // heads per lane in flight of the wave-per-token kernel (2, 4, 6, 8)
    int rope_wgs_per_cu = 0; // wave-per-token kernel: persistent grid of this many workgroups per CU (0: one token per wave)
    int rope_nx = 0;         // NeoX 128 kernel of 8 lanes per head: 0 auto, -1 never, 1..3 always with that many passes per wave
    int rope_nx_run = 0;     // ... consecutive items of one wave (a token's angles evaluated once per run; 0 auto)
    int rope_ss32 = 0;       // ... head norm's sum of squares in fp32 (1) instead of fp64
    int sample_rows_min = 0; // argmax / Gumbel: rows from which a workgroup owns a row (0: 512)
    int sample_threads = 0;  // ... and its lanes (256, 512, 1024; 0: 256)
    int had_unroll = 0;      // Hadamard: 128-blocks per 16-lane group (1, 2, 4; 0: 1)
    int had_mfma_unroll = 0; // matrix-core Hadamard kernels: spans (act-mul: rows of a span) per wave in flight (1, 2, 4; 0: 2)
    int had_mfma_per_cu = 0; // ... workgroups per CU of a looping grid (0: the kernel's default; < 0: one item per wave, no cap)
    int had_threads = 0;     // lanes per workgroup of k_had, k_had_mfma and k_act_mul_had_mfma (64, 128, 256; 0: the default)
    int embed_threads = 0;
};
#ifdef EXL3R_TUNING
Tuning& tuning();
#else
inline const Tuning& tuning()
{
    static constexpr Tuning t{};
    return t;
}
#endif

// Lanes per workgroup of the Hadamard kernels (k_had, k_had_mfma, k_act_mul_had_mfma): one wave.  Same
// process, orders rotated, us for 64 / 128 / 256 lanes: had_r_128 [8192, 5120] butterfly 29.95 / 31.72 /
// 31.79, matrix cores 29.85 / 30.14 / 30.15; SiLU -> rotation [8192, 17408] 130.7 / 131.6 / 130.4; the
// MLP tail from raw gate / up 142.1 / 144.8 / 146.2; 64 against 256 lanes, alternating: the MLP tail at
// [4096, 25600] 104.6 against 107.1, the Qwen3-32B prefill layer's row ops 308.2 against 310.5.
inline int had_threads()
{
    const int t = tuning().had_threads;
    return t == 64 || t == 128 || t == 256 ? t : 64;
}

// Compute units of the current device (cached after the first call).
int device_cus();

}  // namespace exl3r
