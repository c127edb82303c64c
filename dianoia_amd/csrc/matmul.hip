// dnx_matmul_q8 / dnx_matmul_q4: one matmul command's product route on
// device pointers (the kernels lab_gpu_enc_matmul_* runs at commit; the
// route itself is in matmul_route.h).
#include "dnx_kernels.h"
#include "matmul_route.h"

extern "C" {

int64_t dnx_matmul_workspace_bytes(int64_t cols, int64_t n) {
  return dnx::matmul_workspace_bytes(cols, n);
}

int dnx_matmul_q8(const int8_t* qs, const float* scales, const float* x, float* y, int64_t rows,
                  int64_t cols, int64_t n, int int8_inputs, void* workspace,
                  int64_t workspace_bytes, dnx_stream_t stream) {
  return dnx::matmul_route(false, qs, scales, x, y, rows, cols, n, int8_inputs != 0, workspace,
                           workspace_bytes, (hipStream_t)stream, [](dnx::MatmulStep) {});
}

int dnx_matmul_q4(const uint8_t* qs, const uint16_t* scales, const float* x, float* y,
                  int64_t rows, int64_t cols, int64_t n, int int8_inputs, void* workspace,
                  int64_t workspace_bytes, dnx_stream_t stream) {
  return dnx::matmul_route(true, qs, scales, x, y, rows, cols, n, int8_inputs != 0, workspace,
                           workspace_bytes, (hipStream_t)stream, [](dnx::MatmulStep) {});
}

}  // extern "C"
