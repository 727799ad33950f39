// Device-side helpers shared by the gfx950 kernels: wave reductions, nibble
// unpacking, the exact int4/E2M1 decodes and the per-token int8 quantizer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lbk {

constexpr int kWave = 64;      // CDNA wavefront width
constexpr int kGroup = 128;    // int4 group (elements)
constexpr int kMxBlock = 32;   // MXFP4 block (elements)

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

// Sum over each 32-lane half of the wave (the xor offsets never cross lane 32).
__device__ __forceinline__ int half_wave_sum(int v) {
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// Low / high nibbles of the four bytes of w, each in its own byte (values 0..15).
__device__ __forceinline__ uint32_t lo_nibbles(uint32_t w) { return w & 0x0F0F0F0Fu; }
__device__ __forceinline__ uint32_t hi_nibbles(uint32_t w) { return (w >> 4) & 0x0F0F0F0Fu; }

// Bytes (n - z) as two's-complement int8 for four nibble bytes n (0..15) and a
// zero-point z (0..15): (n | 0x80) - z stays in [113, 143] so no borrow crosses a
// byte, and flipping bit 7 back gives (n - z) mod 256.
__device__ __forceinline__ uint32_t sub_zero_bytes(uint32_t nib, uint32_t zrep) {
  return ((nib | 0x80808080u) - zrep) ^ 0x80808080u;
}

// E8M0 exponent byte -> float32 scale 2^(e-127); 0 -> 2^-127 (subnormal), 255 -> NaN.
__device__ __forceinline__ float e8m0_to_f32(uint32_t e) {
  const uint32_t bits = e == 0 ? 0x00400000u : (e == 255 ? 0x7FC00000u : e << 23);
  return __uint_as_float(bits);
}

// E2M1 values of the two nibbles of byte `sel` of w: .x = low nibble, .y = high
// nibble, times `scale` (a power of two, so the product is exact).
template <int SEL>
__device__ __forceinline__ v2f e2m1_pair(uint32_t w, float scale) {
  return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, scale, SEL);
}

// ---------------------------------------------------------------- int8 quantizer
//
// Per-token symmetric quantization, bit-identical to the reference
// (src/lowbit/csrc/dispatch.c:231-257): amax = max |x| (NaN never wins, as with
// the reference's `a > amax`), sc = amax / 127 with IEEE float32 division (1 if
// amax == 0), q = clamp(rint(x / sc), -127, 127) with round-half-to-even.

__device__ __forceinline__ int8_t quant_one(float v, float sc) {
  float q = rintf(v / sc);
  q = q > 127.0f ? 127.0f : (q < -127.0f ? -127.0f : q);
  return (int8_t)(int)q;
}

// Four consecutive elements -> packed int8x4 and their integer sum.
__device__ __forceinline__ uint32_t quant4(float4 v, float sc, int &sum) {
  const int8_t a = quant_one(v.x, sc), b = quant_one(v.y, sc);
  const int8_t c = quant_one(v.z, sc), d = quant_one(v.w, sc);
  sum = (int)a + (int)b + (int)c + (int)d;
  return (uint32_t)(uint8_t)a | ((uint32_t)(uint8_t)b << 8) |
         ((uint32_t)(uint8_t)c << 16) | ((uint32_t)(uint8_t)d << 24);
}

// amax of one row of Kp floats (Kp % 4 == 0) by a block of NT threads; `red` is
// LDS scratch of NT/64 floats. Every thread gets the result.
template <int NT>
__device__ __forceinline__ float block_row_amax(const float *__restrict__ xr, int Kp, float *red) {
  float amax = 0.0f;
  for (int i = threadIdx.x * 4; i < Kp; i += NT * 4) {
    const float4 v = *reinterpret_cast<const float4 *>(xr + i);
    amax = fmaxf(amax, fabsf(v.x));
    amax = fmaxf(amax, fabsf(v.y));
    amax = fmaxf(amax, fabsf(v.z));
    amax = fmaxf(amax, fabsf(v.w));
  }
  amax = wave_max(amax);
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = amax;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < NT / kWave; w++) r = fmaxf(r, red[w]);
  __syncthreads();  // red may be reused by the caller
  return r;
}

__device__ __forceinline__ float row_scale(float amax) {
  return amax > 0.0f ? amax / 127.0f : 1.0f;
}

}  // namespace lbk
