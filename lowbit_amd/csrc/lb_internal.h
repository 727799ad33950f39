// Host-side launch interface between the C ABI (lb_api.hip) and the gfx950
// kernels (lb_kernels.hip). Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace lbk {

enum Fmt { F_W4A16 = 0, F_MXFP4 = 1, F_W4A8 = 2, F_W4A8Q = 3 };

// Operands of one GEMM; unused pointers are null. All pointers are device memory.
struct GemmArgs {
  const float *x = nullptr;       // [M, Kp] fp32 (W4A16, MXFP4, W4A8)
  const int8_t *xq = nullptr;     // [M, Kp] int8 (W4A8Q)
  const float *xs = nullptr;      // [M] (W4A8Q)
  const int32_t *asum = nullptr;  // [M, Kp/128] (W4A8Q)
  const uint8_t *qw = nullptr;    // [N, Kp/2]
  const float *scales = nullptr;  // [N, Kp/128]
  const uint8_t *zeros = nullptr; // [N, Kp/128] or null (z = 8)
  const uint8_t *e8m0 = nullptr;  // [N, Kp/32]
  float *y = nullptr;             // [M, N]
  int M = 0, Kp = 0, N = 0;
  bool tiled = false;             // xq / asum in the tiled layout of the MFMA path
};

// Small-M VALU kernels: largest M they take and the LDS they need.
constexpr int kGemvMaxM = 4;
constexpr size_t kGemvLdsLimit = 60 * 1024;  // dynamic LDS, leaving room for static scratch
size_t gemv_lds_bytes(int fmt, int M, int Kp);
bool gemv_eligible(int fmt, int M, int Kp);

hipError_t launch_gemv(int fmt, const GemmArgs &a, int num_cus, hipStream_t s);
// Per-token int8 quantizer: xq, xs, asum as lb_quant_act_int8, or (tiled) xq and asum
// in the MFMA path's tiled layout over ceil(M/16)*16 rows, padding rows zero.
hipError_t launch_quant(const float *x, int M, int Kp, int8_t *xq, float *xs, int32_t *asum, bool tiled,
                        hipStream_t s);
// Bytes of the tiled xq / asum for M rows.
inline size_t tiled_xq_bytes(int M, int Kp) { return (size_t)((M + 15) / 16) * 16 * Kp; }
inline size_t tiled_asum_bytes(int M, int Kp) { return (size_t)((M + 15) / 16) * 16 * (Kp / 128) * 4; }
// int8 MFMA W4A8 on quantized activations; with `out` non-null it writes the
// exact int32 group accumulators [M, N, G] instead of Y.
hipError_t launch_w4a8_mfma(const GemmArgs &a, int32_t *out, int num_cus, hipStream_t s);
// fp32 MFMA W4A16 / MXFP4.
hipError_t launch_f32_mfma(int fmt, const GemmArgs &a, hipStream_t s);
// exact int32 group accumulators through the VALU dot4 arithmetic of the GEMV.
hipError_t launch_groupacc_dot4(const int8_t *xq, const int32_t *asum, int M, int Kp,
                                const uint8_t *qw, const uint8_t *zeros, int N,
                                int32_t *out, hipStream_t s);
hipError_t launch_copy(void *dst, const void *src, size_t bytes, hipStream_t s);

}  // namespace lbk
