// Internal launchers shared between translation units (no argument checks;
// the extern "C" entry points validate before calling them).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/wf_api.h"

namespace wf {

// gelu: quantize bf16(gelu_tanh(x)) in place of x.
int launch_quant_rows_i8(const void* x, int64_t M, int64_t K, int64_t ldx, int8_t* q, int64_t ldq, float* scales,
                         hipStream_t stream, bool gelu = false);

int launch_gemm_i8(const int8_t* a, const int8_t* w, int64_t M, int64_t N, int64_t K, const float* sx,
                   const float* sw, const void* bias, void* y, int64_t ldy, int32_t* acc_out, int gelu,
                   hipStream_t stream);

int launch_gemm_fp8_pertensor(const uint8_t* a, const uint8_t* w, int64_t M, int64_t N, int64_t K,
                              const float* a_scale, const float* w_scale, const void* bias, void* y, int64_t ldy,
                              hipStream_t stream);

int launch_fp8_quant_pertensor(const void* x, int64_t rows, int64_t k, int64_t ldx, int mode, uint8_t* codes,
                               float* scale, float* partials, hipStream_t stream);

}  // namespace wf
