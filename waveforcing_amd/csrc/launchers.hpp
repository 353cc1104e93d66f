// Internal launchers shared between translation units (no argument checks;
// the extern "C" entry points validate before calling them).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wf {

int launch_quant_rows_i8(const void* x, int64_t M, int64_t K, int64_t ldx, int8_t* q, int64_t ldq, float* scales,
                         hipStream_t stream);

int launch_gemm_i8(const int8_t* a, const int8_t* w, int64_t M, int64_t N, int64_t K, const float* sx,
                   const float* sw, const void* bias, void* y, int64_t ldy, int32_t* acc_out, int gelu,
                   hipStream_t stream);

}  // namespace wf
