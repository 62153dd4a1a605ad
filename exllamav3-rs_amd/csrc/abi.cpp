// Thread-local error reporting and the version entry point of the C ABI; with EXL3R_TUNING (the
// sweep/test build only) also the launch-shape overrides of csrc/tuning.h.
#include "abi.hpp"
#ifdef EXL3R_TUNING
#include "tuning.h"
#endif

#include <cstdarg>
#include <cstdio>

namespace exl3r {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

int launch_status(const char* op)
{
    const hipError_t e = t_launch_error;
    if (e != hipSuccess) return set_error((int)e, "%s: kernel launch failed: %s", op, hipGetErrorString(e));
    return EXL3R_OK;
}

const char* dtype_name(int dt)
{
    switch (dt)
    {
        case EXL3R_F32: return "f32";
        case EXL3R_F16: return "f16";
        case EXL3R_BF16: return "bf16";
        case EXL3R_I32: return "i32";
        case EXL3R_I64: return "i64";
        default: return "?";
    }
}

#ifdef EXL3R_TUNING
Tuning& tuning()
{
    static Tuning t;
    return t;
}
#endif

int device_cus()
{
    static int n = 0;
    if (n == 0)
    {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            n = v;
        else
            n = 256;
    }
    return n;
}

}  // namespace exl3r

extern "C" int exl3r_version(void) { return 10000; }

extern "C" const char* exl3r_last_error(void) { return exl3r::g_last_error; }

#ifdef EXL3R_TUNING
extern "C" void exl3r_tune_rms(int maxv, int threads)
{
    exl3r::tuning().rms_maxv = maxv;
    exl3r::tuning().rms_threads = threads;
}

extern "C" void exl3r_tune_rms_rows(int rows_per_lane) { exl3r::tuning().rms_rows_rpl = rows_per_lane; }

extern "C" void exl3r_tune_rms_split(int split, int wmode)
{
    exl3r::tuning().rms_split = split;
    exl3r::tuning().rms_split_wm = wmode;
}

extern "C" void exl3r_tune_rms_mode(int sum32, int wmode, int r_cached, int pipe)
{
    exl3r::tuning().rms_sum32 = sum32;
    exl3r::tuning().rms_wmode = wmode;
    exl3r::tuning().rms_r_cached = r_cached;
    exl3r::tuning().rms_pipe = pipe;
}

extern "C" void exl3r_tune_act(int unroll, int threads, int blocks_per_cu)
{
    exl3r::tuning().act_unroll = unroll;
    exl3r::tuning().act_threads = threads;
    exl3r::tuning().act_blocks_per_cu = blocks_per_cu;
}

extern "C" void exl3r_tune_rope(int iters) { exl3r::tuning().rope_iters = iters; }
extern "C" void exl3r_tune_rope_tok(int use, int hpl, int wgs_per_cu)
{
    exl3r::tuning().rope_tok = use;
    exl3r::tuning().rope_hpl = hpl;
    exl3r::tuning().rope_wgs_per_cu = wgs_per_cu;
}

extern "C" void exl3r_tune_rope_nx(int passes) { exl3r::tuning().rope_nx = passes; }
extern "C" void exl3r_tune_rope_nx_run(int run) { exl3r::tuning().rope_nx_run = run; }
extern "C" void exl3r_tune_rope_ss32(int on) { exl3r::tuning().rope_ss32 = on; }

extern "C" void exl3r_tune_sample(int rows_min, int threads)
{
    exl3r::tuning().sample_rows_min = rows_min;
    exl3r::tuning().sample_threads = threads;
}

extern "C" void exl3r_tune_had(int blocks_per_group) { exl3r::tuning().had_unroll = blocks_per_group; }

extern "C" void exl3r_tune_had_mfma(int unroll, int blocks_per_cu)
{
    exl3r::tuning().had_mfma_unroll = unroll;
    exl3r::tuning().had_mfma_per_cu = blocks_per_cu;
}

extern "C" void exl3r_tune_had_threads(int threads) { exl3r::tuning().had_threads = threads; }

extern "C" void exl3r_tune_embed(int threads) { exl3r::tuning().embed_threads = threads; }
#endif  // EXL3R_TUNING
