// Weight quantizers on the device: fp32 [N, K] row-major in HBM -> the public packed
// int4 (groups of 128, or 32) and MXFP4 formats, byte for byte what the host packers produce
// (src/lowbit/formats.py:90-142 and :182-212). A model's weights are uploaded once as
// fp32 and packed where they will be read, instead of on the host.
//
// Packed layouts (src/lowbit/csrc/lowbit.h:9-19): inside each block (128 int4 codes,
// 32 E2M1 codes) byte j holds element j in its low nibble and element j + block/2 in
// its high nibble; K is padded to a whole block and padded elements get the code that
// decodes to 0.
//
// Bit-exactness: every division is IEEE float32 (the build keeps fp32 division
// correctly rounded and denormals), rint is round-half-to-even, and reductions are
// max / min / first-index selections, which do not depend on the order of combining.
#include <math.h>

#include "lb_device.h"
#include "lb_internal.h"

namespace lbk {

constexpr int kQT = 256;  // 4 waves per workgroup, one group (or 4 MX blocks) per wave

__device__ __forceinline__ float xor_max(float v, int w) { return fmaxf(v, __shfl_xor(v, w)); }
__device__ __forceinline__ float xor_min(float v, int w) { return fminf(v, __shfl_xor(v, w)); }

// int4, groups of GS = 128 or 32 elements: L = GS / 2 lanes per group, 64 / L groups
// per wave; lane j of a group holds elements j and j + GS / 2, exactly the two
// nibbles of packed byte j of the group (the "j / j+half" layout).
//   absmax:     s = max|w| / 7,          q = clip(rint(w / s), -8, 7) + 8
//   signed-max: s = m / -8 (m = the first element of largest magnitude, sign kept)
//   asym:       s = (max(w, 0) - min(w, 0)) / 15, z = clip(rint(-min / s), 0, 15),
//               q = clip(rint(w / s) + z, 0, 15)
// A scale that is not > 0 (absmax, asym) or is 0 (signed-max) becomes 1.
template <int MODE, int GS>  // MODE 0 absmax, 1 signed-max, 2 asym
__global__ __launch_bounds__(kQT) void quantize_int4_kernel(const float *__restrict__ w, int N, int K, int G,
                                                             uint8_t *__restrict__ qw, float *__restrict__ scales,
                                                             uint8_t *__restrict__ zeros) {
  constexpr int L = GS / 2, GPW = kWave / L;
  const int lane = threadIdx.x & (kWave - 1);
  const int GQ = (G + GPW - 1) / GPW;  // wave items per row
  const long long item = (long long)blockIdx.x * (kQT / kWave) + threadIdx.x / kWave;
  if (item >= (long long)N * GQ) return;  // whole waves only: no barrier below
  const int row = (int)(item / GQ), g = (int)(item % GQ) * GPW + lane / L, j = lane % L;
  const bool live = g < G;  // the last item of a row may hold groups past the row
  const int k0 = g * GS + j, k1 = k0 + L;
  const float *wr = w + (size_t)row * K;
  const bool in0 = live && k0 < K, in1 = live && k1 < K;
  const float x0 = in0 ? wr[k0] : 0.0f, x1 = in1 ? wr[k1] : 0.0f;
  float s, zf = 8.0f, lo_q = -8.0f, hi_q = 7.0f;
  // xor offsets below L keep every reduction inside one group's lanes
  if (MODE == 2) {
    float hi = fmaxf(x0, x1), lo = fminf(x0, x1);
    for (int o = L / 2; o > 0; o >>= 1) hi = xor_max(hi, o), lo = xor_min(lo, o);
    hi = fmaxf(hi, 0.0f);
    lo = fminf(lo, 0.0f);
    s = (hi - lo) / 15.0f;
    s = s > 0.0f ? s : 1.0f;
    zf = fminf(fmaxf(__builtin_rintf(-lo / s), 0.0f), 15.0f);
    lo_q = 0.0f;
    hi_q = 15.0f;
  } else if (MODE == 1) {
    // first element of largest magnitude: larger |x|, then the smaller index
    float a = fabsf(x0), m = x0;
    int ix = k0;
    if (fabsf(x1) > a) a = fabsf(x1), m = x1, ix = k1;
    for (int o = L / 2; o > 0; o >>= 1) {
      const float oa = __shfl_xor(a, o), om = __shfl_xor(m, o);
      const int oi = __shfl_xor(ix, o);
      if (oa > a || (oa == a && oi < ix)) a = oa, m = om, ix = oi;
    }
    s = m / -8.0f;
    s = s != 0.0f ? s : 1.0f;
  } else {
    float a = fmaxf(fabsf(x0), fabsf(x1));
    for (int o = L / 2; o > 0; o >>= 1) a = xor_max(a, o);
    s = a / 7.0f;
    s = s > 0.0f ? s : 1.0f;
  }
  // symmetric: code = clip(rint(w / s), -8, 7) + 8; asym: clip(rint(w / s) + z, 0, 15)
  const float add = MODE == 2 ? zf : 0.0f, off = MODE == 2 ? 0.0f : 8.0f;
  const float c0 = fminf(fmaxf(__builtin_rintf(x0 / s) + add, lo_q), hi_q) + off;
  const float c1 = fminf(fmaxf(__builtin_rintf(x1 / s) + add, lo_q), hi_q) + off;
  const uint32_t pad = (uint32_t)zf;  // padded elements decode to 0
  const uint32_t q0 = in0 ? (uint32_t)c0 : pad, q1 = in1 ? (uint32_t)c1 : pad;
  if (!live) return;
  qw[(size_t)row * ((size_t)G * L) + (size_t)g * L + j] = (uint8_t)(q0 | (q1 << 4));
  if (j == 0) {
    scales[(size_t)row * G + g] = s;
    if (MODE == 2) zeros[(size_t)row * G + g] = (uint8_t)pad;
  }
}

// E2M1 code of v (already divided by the block scale): round to nearest, ties to the
// even mantissa code, saturating at +-6; the magnitude code counts the decision
// points below |v| (ties at .25, 1.25, 2.5, 5 round down, at .75, 1.75, 3.5 up).
// -0 and values that round to 0 give code 0.
__device__ __forceinline__ uint32_t e2m1_code(float v) {
  const float a = fabsf(v);
  const uint32_t mag = (uint32_t)(a > 0.25f) + (uint32_t)(a >= 0.75f) + (uint32_t)(a > 1.25f) +
                       (uint32_t)(a >= 1.75f) + (uint32_t)(a > 2.5f) + (uint32_t)(a >= 3.5f) + (uint32_t)(a > 5.0f);
  return mag | ((signbit(v) && mag) ? 8u : 0u);
}

// MXFP4: one wave per 128 elements of a row = 4 blocks of 32; the 16 lanes of row
// b (lanes 16b .. 16b + 15) own block b, lane j holding elements j and j + 16, the
// two nibbles of packed byte j. Shared exponent (OCP MX v1.0): e = floor(log2(amax))
// - 2 + 127 clipped to [0, 254] (127 for an all-zero block), scale 2^(e - 127).
// log2 is the float32 log2 correctly rounded (double log2, rounded once to float32):
// just below a power of two it rounds up to the integer, and the host packer's
// float32 log2 does the same there (the only place where the floor can differ).
__global__ __launch_bounds__(kQT) void quantize_mxfp4_kernel(const float *__restrict__ w, int N, int K, int Kp,
                                                              int C, uint8_t *__restrict__ qw,
                                                              uint8_t *__restrict__ e8m0) {
  const int lane = threadIdx.x & (kWave - 1);
  const long long item = (long long)blockIdx.x * (kQT / kWave) + threadIdx.x / kWave;
  if (item >= (long long)N * C) return;
  const int row = (int)(item / C), chunk = (int)(item % C);
  const int b = lane >> 4, j = lane & 15;
  const int blk = chunk * 4 + b;  // block index in the row
  const bool live = blk * 32 < Kp;
  const int k0 = blk * 32 + j, k1 = k0 + 16;
  const float *wr = w + (size_t)row * K;
  const float x0 = (live && k0 < K) ? wr[k0] : 0.0f, x1 = (live && k1 < K) ? wr[k1] : 0.0f;
  float a = fmaxf(fabsf(x0), fabsf(x1));
  for (int o = 8; o > 0; o >>= 1) a = xor_max(a, o);  // within the 16-lane row
  int e = 127;
  if (a > 0.0f) {
    const float lg = (float)log2((double)a);
    const int sh = (int)floorf(lg) - 2 + 127;
    e = sh < 0 ? 0 : (sh > 254 ? 254 : sh);
  }
  if (!live) return;
  const float scale = e == 0 ? 0x1p-127f : __uint_as_float((uint32_t)e << 23);
  const uint32_t q0 = e2m1_code(x0 / scale), q1 = e2m1_code(x1 / scale);
  const int nb = Kp / 32;
  qw[(size_t)row * (Kp / 2) + blk * 16 + j] = (uint8_t)(q0 | (q1 << 4));
  if (j == 0) e8m0[(size_t)row * nb + blk] = (uint8_t)e;
}

static unsigned waves_grid(long long items) { return (unsigned)((items + kQT / kWave - 1) / (kQT / kWave)); }

template <int GS>
static void launch_quantize_int4_g(const float *w, int N, int K, int mode, uint8_t *qw, float *scales, uint8_t *zeros,
                                   hipStream_t s) {
  const int G = (K + GS - 1) / GS, GPW = kWave / (GS / 2);
  const dim3 grid(waves_grid((long long)N * ((G + GPW - 1) / GPW))), block(kQT);
  if (mode == 2)
    hipLaunchKernelGGL((quantize_int4_kernel<2, GS>), grid, block, 0, s, w, N, K, G, qw, scales, zeros);
  else if (mode == 1)
    hipLaunchKernelGGL((quantize_int4_kernel<1, GS>), grid, block, 0, s, w, N, K, G, qw, scales, zeros);
  else
    hipLaunchKernelGGL((quantize_int4_kernel<0, GS>), grid, block, 0, s, w, N, K, G, qw, scales, zeros);
}

hipError_t launch_quantize_int4(const float *w, int N, int K, int mode, int group, uint8_t *qw, float *scales,
                                uint8_t *zeros, hipStream_t s) {
  if (group == 128)
    launch_quantize_int4_g<128>(w, N, K, mode, qw, scales, zeros, s);
  else if (group == 32)
    launch_quantize_int4_g<32>(w, N, K, mode, qw, scales, zeros, s);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_quantize_mxfp4(const float *w, int N, int K, uint8_t *qw, uint8_t *e8m0, hipStream_t s) {
  const int Kp = (K + 31) / 32 * 32, C = (Kp + 127) / 128;
  hipLaunchKernelGGL(quantize_mxfp4_kernel, dim3(waves_grid((long long)N * C)), dim3(kQT), 0, s, w, N, K, Kp, C, qw,
                     e8m0);
  return hipGetLastError();
}

}  // namespace lbk
