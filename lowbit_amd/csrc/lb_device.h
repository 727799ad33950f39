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
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- reductions
//
// Cross-lane steps use DPP (data-parallel primitives: a VALU operand read from
// another lane) instead of LDS permutes, so each step costs one VALU op:
//   quad_perm [1,0,3,2], [2,3,0,1]  -> every lane holds its quad's total
//   row_half_mirror, row_mirror     -> every lane holds its 16-lane row's total
//   row_bcast:15 (rows 1, 3)        -> rows 1 / 3 hold rows 0+1 / 2+3
//   row_bcast:31 (rows 2, 3)        -> row 3 holds the wave total
// Rows excluded by the row mask add the identity (`old` operand).
constexpr int kDppQuad1032 = 0xB1, kDppQuad2301 = 0x4E, kDppRowHalfMirror = 0x141,
              kDppRowMirror = 0x140, kDppRowBcast15 = 0x142, kDppRowBcast31 = 0x143;

template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ float dpp_f(float v, float identity) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(identity), __float_as_int(v), CTRL, ROWS, 0xF, false));
}
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ int dpp_i(int v, int identity) {
  return __builtin_amdgcn_update_dpp(identity, v, CTRL, ROWS, 0xF, false);
}

// Sum over the wave; every lane gets the total (read back from lane 63).
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<kDppQuad1032>(v, 0.0f);
  v += dpp_f<kDppQuad2301>(v, 0.0f);
  v += dpp_f<kDppRowHalfMirror>(v, 0.0f);
  v += dpp_f<kDppRowMirror>(v, 0.0f);
  v += dpp_f<kDppRowBcast15, 0xA>(v, 0.0f);
  v += dpp_f<kDppRowBcast31, 0xC>(v, 0.0f);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Max over the wave (NaN never wins, as with fmaxf); every lane gets it.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f<kDppQuad1032>(v, v));
  v = fmaxf(v, dpp_f<kDppQuad2301>(v, v));
  v = fmaxf(v, dpp_f<kDppRowHalfMirror>(v, v));
  v = fmaxf(v, dpp_f<kDppRowMirror>(v, v));
  v = fmaxf(v, dpp_f<kDppRowBcast15, 0xA>(v, v));
  v = fmaxf(v, dpp_f<kDppRowBcast31, 0xC>(v, v));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Lane `lane` (wave-uniform) of v takes the wave-uniform value `bits`; the other
// lanes keep theirs: v_writelane_b32 through LLVM's intrinsic, which clang exposes
// as no builtin. The compiler then sets M0 for the lane select itself (gfx9 reads
// one scalar register per VALU instruction) and knows that M0 changes.
__device__ int lb_writelane_i32(int val, int lane, int old) __asm("llvm.amdgcn.writelane.i32");
__device__ __forceinline__ void write_lane(float &v, int bits, int lane) {
  v = __int_as_float(lb_writelane_i32(bits, lane, __float_as_int(v)));
}

// Max over the wave of 64-bit keys (unsigned); every lane gets it. Each step moves
// both halves by the same DPP pattern; lanes the pattern leaves out read 0, which
// is below every key.
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ unsigned long long dpp_u64(unsigned long long v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, ROWS, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, ROWS, 0xF, false);
  return ((unsigned long long)hi << 32) | lo;
}
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
  unsigned long long o;
  o = dpp_u64<kDppQuad1032>(v);
  v = o > v ? o : v;
  o = dpp_u64<kDppQuad2301>(v);
  v = o > v ? o : v;
  o = dpp_u64<kDppRowHalfMirror>(v);
  v = o > v ? o : v;
  o = dpp_u64<kDppRowMirror>(v);
  v = o > v ? o : v;
  o = dpp_u64<kDppRowBcast15, 0xA>(v);
  v = o > v ? o : v;
  o = dpp_u64<kDppRowBcast31, 0xC>(v);
  v = o > v ? o : v;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, 63);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), 63);
  return ((unsigned long long)hi << 32) | lo;
}

// Sum over each 32-lane half of the wave; the totals land in lanes 31 and 63
// (other lanes hold partial sums).
__device__ __forceinline__ int half_wave_sum(int v) {
  v += dpp_i<kDppQuad1032>(v, 0);
  v += dpp_i<kDppQuad2301>(v, 0);
  v += dpp_i<kDppRowHalfMirror>(v, 0);
  v += dpp_i<kDppRowMirror>(v, 0);
  v += dpp_i<kDppRowBcast15, 0xA>(v, 0);
  return v;
}

// Float sum over each 32-lane half of the wave; the totals land in lanes 31 and 63.
__device__ __forceinline__ float half_wave_sum_f(float v) {
  v += dpp_f<kDppQuad1032>(v, 0.0f);
  v += dpp_f<kDppQuad2301>(v, 0.0f);
  v += dpp_f<kDppRowHalfMirror>(v, 0.0f);
  v += dpp_f<kDppRowMirror>(v, 0.0f);
  v += dpp_f<kDppRowBcast15, 0xA>(v, 0.0f);
  return v;
}

// Sum over each group of eight lanes; every lane of the group gets it (quad sums,
// then the mirrored quad of the same half-row).
__device__ __forceinline__ int eighth_wave_sum(int v) {
  v += dpp_i<kDppQuad1032>(v, 0);
  v += dpp_i<kDppQuad2301>(v, 0);
  v += dpp_i<kDppRowHalfMirror>(v, 0);
  return v;
}

// ---------------------------------------------------------------- buffer loads
//
// Raw buffer loads through a resource descriptor (base, byte count): offsets at
// or past the byte count read 0 in hardware, so a descriptor per weight row
// makes row and chunk tails free of clamps and selects. Offsets are 32-bit
// (rows and activation vectors are far below 4 GiB). The third descriptor word
// 0x00020000 is the raw-buffer format word of the gfx9 family.
typedef __amdgpu_buffer_rsrc_t Rsrc;

__device__ __forceinline__ Rsrc make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 ld_b128(Rsrc r, uint32_t off) {
  const v4u v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}
// the same with cache-policy bits AUX (2: non-temporal, for data read once)
template <int AUX>
__device__ __forceinline__ uint4 ld_b128_aux(Rsrc r, uint32_t off) {
  const v4u v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, AUX);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float4 ld_f4(Rsrc r, uint32_t off) {
  const v4u v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}
__device__ __forceinline__ float ld_f32(Rsrc r, uint32_t off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
}
__device__ __forceinline__ uint32_t ld_u32(Rsrc r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}
__device__ __forceinline__ uint32_t ld_u8(Rsrc r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b8(r, (int)off, 0, 0);
}
// With a workgroup-uniform part `soff` in the instruction's scalar offset, so that
// loads at several uniform distances share one vector offset register. The
// hardware range check covers the vector offset only: soff must keep the access
// inside the buffer.
__device__ __forceinline__ uint4 ld_b128(Rsrc r, uint32_t voff, uint32_t soff) {
  const v4u v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float ld_f32(Rsrc r, uint32_t voff, uint32_t soff) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0));
}
__device__ __forceinline__ uint32_t ld_u32(Rsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0);
}

// Hides a value from the optimizer (no instruction is emitted), so that a mask
// is not folded into later byte extractions: (m >> 8k) & 0xFF of an opaque m
// becomes one v_cvt_f32_ubyte<k> instead of a bitfield extract plus a convert.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm("" : "+v"(v));
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

// ---------------------------------------------------------------- bf16 terms
//
// Round-to-nearest-even of x to bf16, returned as the float32 bit pattern with the
// low 16 bits clear (so it is also the float value of the bf16). Finite x up to the
// largest bf16 below 2^128; NaN stays NaN.
__device__ __forceinline__ uint32_t bf16_rne(float x) {
  const uint32_t u = __float_as_uint(x);
  return (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
}

// x = hi + mid + lo exactly for normal x (each term keeps 8 significant bits and
// each remainder is exact in float32), as three float32 bit patterns.
__device__ __forceinline__ void split3(float x, uint32_t &hi, uint32_t &mid, uint32_t &lo) {
  hi = bf16_rne(x);
  const float r1 = x - __uint_as_float(hi);
  mid = bf16_rne(r1);
  lo = bf16_rne(r1 - __uint_as_float(mid));
}

// Two float32 values whose low 16 bits are zero (or may be dropped exactly) ->
// bf16x2 with `a` in the low half.
__device__ __forceinline__ uint32_t pack_bf16(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
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

// Four consecutive elements -> packed int8x4 (IEEE division for every element).
__device__ __forceinline__ uint32_t quant4(float4 v, float sc) {
  const int8_t a = quant_one(v.x, sc), b = quant_one(v.y, sc);
  const int8_t c = quant_one(v.z, sc), d = quant_one(v.w, sc);
  return (uint32_t)(uint8_t)a | ((uint32_t)(uint8_t)b << 8) |
         ((uint32_t)(uint8_t)c << 16) | ((uint32_t)(uint8_t)d << 24);
}

// Four consecutive elements -> packed int8x4, bit-identical to quant4, without a
// division on the common path. With inv = fl(1/sc), u = fma(v, inv, 128) (one
// rounding) differs from fl(v/sc) + 128 by less than 2^-15:
//   |u - (v*inv + 128)| <= 2^-17 (half an ulp below 256),
//   |v*inv - v/sc| <= |v/sc| * 2^-24 < 2^-17 (|v/sc| <= 127 (1 + 2^-23) since
//   |v| <= amax and sc = fl(amax/127)), and |fl(v/sc) - v/sc| <= 2^-18.
// So unless u lies within 2^-15 of a half-integer, rint(u) - 128 == rint(fl(v/sc))
// (fl(v/sc) is then no tie either), and |u - rint(u)| is exact in float32. rint(u)
// is an integer in [1, 255]: v_cvt_pk_u8_f32 packs it exactly and XOR 0x80 turns
// q + 128 into the two's-complement byte q; the clamp at +-127 can never act.
// A slot with a near-tie, NaN or an overflowed inv (sc < 2^-128) is redone with
// the IEEE division (about one slot in 4000 for random data).
__device__ __forceinline__ uint32_t quant4_fast(float4 v, float sc, float inv) {
  const float u0 = __builtin_fmaf(v.x, inv, 128.0f), u1 = __builtin_fmaf(v.y, inv, 128.0f);
  const float u2 = __builtin_fmaf(v.z, inv, 128.0f), u3 = __builtin_fmaf(v.w, inv, 128.0f);
  const float r0 = __builtin_rintf(u0), r1 = __builtin_rintf(u1);
  const float r2 = __builtin_rintf(u2), r3 = __builtin_rintf(u3);
  constexpr float kSafe = 0.5f - 0x1p-15f;
  const bool ok = ((int)(fabsf(u0 - r0) < kSafe) & (int)(fabsf(u1 - r1) < kSafe) &
                   (int)(fabsf(u2 - r2) < kSafe) & (int)(fabsf(u3 - r3) < kSafe)) != 0;
  uint32_t p = __builtin_amdgcn_cvt_pk_u8_f32(r0, 0, 0u);
  p = __builtin_amdgcn_cvt_pk_u8_f32(r1, 1, p);
  p = __builtin_amdgcn_cvt_pk_u8_f32(r2, 2, p);
  p = __builtin_amdgcn_cvt_pk_u8_f32(r3, 3, p);
  p ^= 0x80808080u;
  if (!ok) p = quant4(v, sc);
  return p;
}

// Sum of the four signed bytes of a packed int8x4.
__device__ __forceinline__ int sum_i8x4(uint32_t p) {
  return __builtin_amdgcn_sdot4((int)p, 0x01010101, 0, false);
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

// fl(a / 127) for a >= 0: one multiply and two fused multiply-adds instead of the IEEE
// division sequence. q0 = fl(a * fl(1/127)), r = a - 127 q0 (exact), q0 + r fl(1/127)
// rounded once; equal to the IEEE quotient for every finite float32 a >= 0. Host and
// device compile the same code: tests/csrc/div127_exhaustive.hip checks every such a
// on the CPU, lbd_probe_div127 on the GPU, both against a / 127.0f. +inf takes the
// division.
__host__ __device__ __forceinline__ float div127(float a) {
  constexpr float kR = 1.0f / 127.0f;
  const float q0 = a * kR;
  const float q1 = __builtin_fmaf(__builtin_fmaf(-q0, 127.0f, a), kR, q0);
  return a <= 3.4028234663852886e38f ? q1 : a / 127.0f;
}

// ---------------------------------------------------------------- argmax keys
//
// (value, index) as one unsigned 64-bit key whose unsigned order is numpy's
// argmax order: any NaN above every number, then larger values, then the smaller
// index. The high word maps the float's bits to an unsigned order (-0 counts as
// +0, as numpy compares them equal), the low word is 0xFFFFFFFF - index. Every
// key is above 0, so 0 means "no value yet" and a 64-bit atomic max combines keys
// from any number of waves.
__device__ __forceinline__ unsigned long long argmax_key(float v, int idx) {
  uint32_t u = __float_as_uint(v);
  uint32_t k;
  if (v != v) {
    k = 0xFFFFFFFFu;
  } else {
    if (v == 0.0f) u = 0;
    k = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  }
  return ((unsigned long long)k << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)idx);
}

__device__ __forceinline__ int argmax_key_index(unsigned long long key) {
  return key ? (int)(0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFull)) : 0;
}

}  // namespace lbk
