// Argument checks shared by the RMSNorm-family entry points (rms_norm.hip, rms_norm_res.hip,
// embedding.hip).
#pragma once

#include <stdint.h>

namespace exl3r {

int check_rms_common(const char* op, const void* x, int xt, int64_t ldx, const void* w, int wt,
                     const void* y, int yt, int64_t ldy, int64_t rows, int64_t dim);

}  // namespace exl3r
