// quant_common.hpp -- host+device pieces of the INT8 calibration epilogue.
//
// Reference: quantize.c:62-81 and 112-129 (the symmetric / affine epilogue
// shared by calibrate_minmax and calibrate_percentile).  The reference build
// converts the rounded zero point with x86 cvttsd2si, which yields INT32_MIN
// for NaN and out-of-range values (e.g. an infinite range gives inf/inf); the
// clamp then maps that to -128.  A plain C++ cast is undefined there, so both
// the device calibrate and the host-side percentile epilogue use this copy.
#pragma once
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "../../include/neural_api.h"

namespace nh {

#define NH_HD __host__ __device__ __forceinline__

// cvttsd2si of an already-rounded double.
NH_HD int32_t x86_cvt_i32(double r)
{
    if (!(r > -2147483649.0 && r < 2147483648.0)) return int32_t(0x80000000u);
    return int32_t(r);
}

NH_HD void minmax_epilogue(double mn, double mx, int symmetric, QuantParams *out)
{
    QuantParams p;
    p.zero_point = 0;
    if (symmetric) {
        double am = fmax(fabs(mn), fabs(mx));
        if (am < 1e-30) am = 1e-30;
        p.scale = am / 127.0;
        p.zero_point = 0;
        p.min_val = -am;
        p.max_val = am;
        p.symmetric = 1;
    } else {
        if (mn == mx) { mn -= 0.5; mx += 0.5; }
        p.scale = (mx - mn) / 255.0;
        if (p.scale < 1e-30) p.scale = 1e-30;
        int32_t zp = x86_cvt_i32(round(-128.0 - mn / p.scale));
        if (zp < -128) zp = -128;
        if (zp > 127) zp = 127;
        p.zero_point = zp;
        p.min_val = mn;
        p.max_val = mx;
        p.symmetric = 0;
    }
    *out = p;
}

}  // namespace nh
