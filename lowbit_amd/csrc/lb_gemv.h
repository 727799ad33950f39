// The small-M GEMV (decode) kernels, shared by the translation units that
// instantiate them: lb_kernels.hip (int4 group 128, MXFP4, W4A8 on quantized
// activations) and lb_gemv_g32.hip (int4 group 32). Device code and launch
// templates only; the host entry points are declared in lb_internal.h.
#pragma once

#include "lb_attn.h"
#include "lb_device.h"
#include "lb_internal.h"

namespace lbk {

// ============================================================ small-M GEMV (VALU)
//
// Decode is a pure HBM stream that lasts a few microseconds; the kernel is built
// around three facts:
//   * every weight byte should be requested as early as possible;
//   * the activation prologue (staging X, or quantizing it for W4A8) is the same
//     for every workgroup, so it should run as few times as possible;
//   * the VALU issue rate, not HBM, is the next limit, so tails and bounds must
//     cost no instructions.
// The grid is persistent: two 512-thread workgroups per CU where two fit at once
// (one elsewhere, see launch_gemv_mb). Each workgroup
// stages (or quantizes) the activations once, and its 8 waves take an even
// share of the weight rows (rows [gw*N/W, (gw+1)*N/W) for global wave gw of W).
// A wave first loads its activation slice into registers, then issues all the
// loads of its first R rows (16 bytes per lane per chunk, plus scales), and only
// then writes the activations to LDS: loads retire in issue order (s_waitcnt
// vmcnt), so the prologue waits for the activations alone while the weight
// stream is in flight. Decode and FMAs run from registers as chunks land, then
// one DPP wave reduction per (activation row, weight row) gives the output.
// All global reads are buffer loads through per-row descriptors: chunks past a
// row's end, rows past the wave's share and activations past Kp read as 0.
//
// Chunk ci of a row is bytes [16ci, 16ci+16) = 32 elements; lane l holds chunks
// ci = l, l + 64, ... (NIT of them; the regime is limited to rows that fit):
//   int4 : group g = ci / 4, bytes b = 16 (ci % 4): low nibbles are elements
//          128g + b + [0,16), high nibbles 128g + 64 + b + [0,16)
//   MXFP4 and int4 with groups of 32: block (group) ci: low nibbles 32ci + [0,16),
//          high nibbles 32ci + 16 + [0,16)
//
// LDS plane layout of the activations: for fp32 X, eight planes of float4,
// plane p = half * 4 + (position within the 16-element half) / 4, entry ci; for
// int8 codes, two planes of 16 bytes (half 0 / 1). Planes hold nchp = nit * 64
// entries (whole steps of 64 chunks), so padding lanes read zeros. Lane reads of
// one plane are consecutive 16-byte words: no bank conflicts.

constexpr int kGemvThreads = 512;
// Cache-policy bits of the GEMVs' weight loads: non-temporal (each weight byte is read
// once per call). At 1 x 11008 x 4096 cold the one-row kernel took 0.3-0.5 us less than
// with the default policy; the LM head (151936 x 896, cold) W4A8 18.8 -> 17.9 us.
constexpr int kWeightAux = 2;
constexpr int kGemvWaves = kGemvThreads / kWave;
constexpr int kGemvMaxNit = 8;   // chunks per lane held in registers (rows up to 16384 elements)
constexpr int kXRegs = 16;       // float4 of activations a thread may hold across the weight loads

__device__ __forceinline__ void chunk_pos(int fmt, int e, int &ci, int &half, int &within) {
  if (fmt == F_MXFP4 || fmt_g32(fmt)) {
    const int r = e & 31;
    ci = e >> 5;
    half = r >> 4;
    within = r & 15;
  } else {
    const int r = e & 127;
    ci = ((e >> 7) << 2) + ((r & 63) >> 4);
    half = r >> 6;
    within = r & 15;
  }
}

inline int gemv_nchp(int Kp) { return ((Kp / 32 + kWave - 1) / kWave) * kWave; }

// Weights of R rows x NIT chunks per lane, with their scales.
template <int F, int R, int NIT>
struct GemvRegs {
  uint4 w[R][NIT];
  float sc[R][NIT];
  int zi[R][NIT];
  // two rows per wave load, int4: the scales and zero-points of the batch's rows,
  // one per lane (lane j: entry j of the rows' contiguous metadata)
  float scb;
  int zb;
};

// Rows rb .. rb+R-1; rows at or past `rend` get zero-length descriptors (read 0).
// HW (rows of at most 32 chunks): slot r holds two rows, rb + 2r in lanes 0..31 and
// rb + 2r + 1 in lanes 32..63, under one descriptor over both (adjacent in memory);
// lanes past a row's chunks read past the descriptor, i.e. zeros.
template <int F, int R, int NIT, bool HW>
__device__ __forceinline__ void gemv_load(const GemmArgs &a, GemvRegs<F, R, NIT> &g, int rb, int rend, int lane,
                                          int nch, int G) {
  static_assert(!HW || NIT == 1, "two rows per wave load: one chunk per lane");
  const uint32_t rowbytes = (uint32_t)(a.Kp >> 1);
  const int zadd = a.zeros ? 0 : 8;  // symmetric weights: z = 8
  constexpr bool kG32 = fmt_g32(F);
  const uint32_t half = HW ? (uint32_t)lane >> 5 : 0u;
  const uint32_t cl = HW ? (uint32_t)lane & 31u : (uint32_t)lane;
  constexpr bool kBatchMeta = HW && F != F_MXFP4;
  if constexpr (kBatchMeta) {
    // the metadata of the batch's 2R rows (at most 2R * 8 <= 64 entries: rows of at
    // most 1024 elements) in one load per array instead of one per slot; gemv_compute
    // hands each lane its own entry by a cross-lane permute
    const uint32_t nb = __builtin_amdgcn_readfirstlane(rb < rend ? min(rend - rb, 2 * R) : 0);
    const size_t rbb = (size_t)__builtin_amdgcn_readfirstlane(nb ? rb : 0);
    const Rsrc rs = make_rsrc(a.scales + rbb * G, nb * (uint32_t)G * 4);
    g.scb = ld_f32(rs, (uint32_t)lane * 4);
    if (a.zeros) {
      const Rsrc rz = make_rsrc(a.zeros + rbb * G, nb * (uint32_t)G);
      g.zb = (int)ld_u8(rz, (uint32_t)lane);
    } else {
      g.zb = zadd;
    }
  }
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int row = rb + (HW ? 2 * r : r);
    // wave-uniform; read back into scalar registers, since the compiler otherwise
    // forms these selects on the vector unit and then loops over the lanes'
    // descriptors one distinct value at a time
    const uint32_t nrows = __builtin_amdgcn_readfirstlane(row < rend ? ((HW && row + 1 < rend) ? 2u : 1u) : 0u);
    const size_t rr = (size_t)__builtin_amdgcn_readfirstlane(nrows ? row : 0);
    const Rsrc rw = make_rsrc(a.qw + rr * rowbytes, nrows * rowbytes);
    if constexpr (F == F_MXFP4) {
      const Rsrc re = make_rsrc(a.e8m0 + rr * nch, nrows * (uint32_t)nch);
#pragma unroll
      for (int it = 0; it < NIT; it++) {
        const uint32_t ci = cl + kWave * it;
        const bool live = !HW || ci < (uint32_t)nch;
        g.w[r][it] = ld_b128_aux<kWeightAux>(rw, live ? half * rowbytes + ci * 16 : 2 * rowbytes);
        g.sc[r][it] = e8m0_to_f32(ld_u8(re, live ? half * (uint32_t)nch + ci : 2 * (uint32_t)nch));
        g.zi[r][it] = 0;
      }
    } else {
      const Rsrc rs = make_rsrc(a.scales + rr * G, nrows * (uint32_t)G * 4);
      const Rsrc rz = make_rsrc(a.zeros ? a.zeros + rr * G : a.qw, a.zeros ? nrows * (uint32_t)G : 0);
#pragma unroll
      for (int it = 0; it < NIT; it++) {
        const uint32_t ci = cl + kWave * it;
        const bool live = !HW || ci < (uint32_t)nch;
        g.w[r][it] = ld_b128_aux<kWeightAux>(rw, live ? half * rowbytes + ci * 16 : 2 * rowbytes);
        if constexpr (kBatchMeta) continue;
        const uint32_t gi = kG32 ? ci : ci >> 2;  // the chunk's group
        g.sc[r][it] = ld_f32(rs, live ? (half * (uint32_t)G + gi) * 4 : 2 * (uint32_t)G * 4);
        g.zi[r][it] = (int)ld_u8(rz, live ? half * (uint32_t)G + gi : 2 * (uint32_t)G) + zadd;
      }
    }
  }
}

// ---- per-chunk arithmetic, shared by gemv_kernel and gemv_paced_kernel so that the
//      two give the same bits

// W4A16: the codes of one 32-bit word of a chunk as float16 pairs of the dequantized
// integers, exactly, for any zero-point z in 0..15. A nibble n masked into the low
// mantissa bits of a half under the exponent of 1024 is the float16 1024 + n (or, left
// in bits 4..7, 1024 + 16 n); subtracting 1024 + z (1024 + 16 z) in float16 is exact
// and leaves n - z (16 (n - z)). Pairs: p0 = (low nibbles of bytes 0, 2), p1 = (high
// nibbles of bytes 0, 2) times 16, p2 = (low nibbles of bytes 1, 3), p3 = (high
// nibbles of bytes 1, 3) times 16. The FMAs then take the half-precision integers
// directly (v_fma_mix_f32: the conversion to fp32 is exact and the FMA rounds once),
// so the products are those of the dequantized weight, as the reference forms them
// (src/lowbit/csrc/kern_scalar.c:10-29), and a row's fp32 rounding stays relative to
// sum |q - z| |x|, the bound's scale, even where a large activation meets a code equal
// to the zero-point (the split sum q x - z sum x rounds relative to sum q |x|).
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
struct W16Zero {
  h2 lo, hi;  // (1024 + z) and (1024 + 16 z), both halves
};
__device__ __forceinline__ W16Zero w4a16_zero(int z) {
  return {__builtin_bit_cast(h2, (0x6400u | (uint32_t)z) * 0x00010001u),
          __builtin_bit_cast(h2, (0x6400u | (uint32_t)(16 * z)) * 0x00010001u)};
}
// (w & mask) | (f & ~mask) in one instruction (v_bfi_b32; the compiler splits the
// constant form into an AND and an OR)
__device__ __forceinline__ uint32_t bit_select(uint32_t mask, uint32_t w, uint32_t f) {
  uint32_t r;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "s"(mask), "v"(w), "v"(f));
  return r;
}
__device__ __forceinline__ void w4a16_pairs(uint32_t w, const W16Zero &zz, h2 (&p)[4]) {
  const uint32_t w8 = w >> 8, e = 0x64006400u;  // e: the exponent of 1024 in both halves
  p[0] = __builtin_bit_cast(h2, bit_select(0x000F000Fu, w, e)) - zz.lo;
  p[1] = __builtin_bit_cast(h2, bit_select(0x00F000F0u, w, e)) - zz.hi;
  p[2] = __builtin_bit_cast(h2, bit_select(0x000F000Fu, w8, e)) - zz.lo;
  p[3] = __builtin_bit_cast(h2, bit_select(0x00F000F0u, w8, e)) - zz.hi;
}

// W4A16: sum_k (q_k - z) x_k of one 16-byte chunk: the low-nibble half in element
// order, then the high-nibble half (accumulated at 16 times its value, then scaled
// back: a power of two, so the same roundings as at its own scale).
__device__ __forceinline__ float w4a16_chunk(uint4 w, const float4 (&xv)[8], int z) {
  const W16Zero zz = w4a16_zero(z);
  const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
  float pl = 0.0f, ph = 0.0f;
#pragma unroll
  for (int d = 0; d < 4; d++) {
    h2 p[4];
    w4a16_pairs(wd[d], zz, p);
    pl = __builtin_fmaf((float)p[0].x, xv[d].x, pl);
    pl = __builtin_fmaf((float)p[2].x, xv[d].y, pl);
    pl = __builtin_fmaf((float)p[0].y, xv[d].z, pl);
    pl = __builtin_fmaf((float)p[2].y, xv[d].w, pl);
    ph = __builtin_fmaf((float)p[1].x, xv[4 + d].x, ph);
    ph = __builtin_fmaf((float)p[3].x, xv[4 + d].y, ph);
    ph = __builtin_fmaf((float)p[1].y, xv[4 + d].z, ph);
    ph = __builtin_fmaf((float)p[3].y, xv[4 + d].w, ph);
  }
  return pl + ph * 0.0625f;
}

// W4A16: the 32 codes of one chunk as exact floats (q - z) for the low-nibble half in
// wl and 16 (q - z) for the high-nibble half in wh (chunk_dot<4> scales that half
// back), for rows used against several activation rows.
__device__ __forceinline__ void w4a16_decode(uint4 w, int z, float (&wl)[16], float (&wh)[16]) {
  const W16Zero zz = w4a16_zero(z);
  const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int d = 0; d < 4; d++) {
    h2 p[4];
    w4a16_pairs(wd[d], zz, p);
    wl[4 * d + 0] = (float)p[0].x; wl[4 * d + 1] = (float)p[2].x;
    wl[4 * d + 2] = (float)p[0].y; wl[4 * d + 3] = (float)p[2].y;
    wh[4 * d + 0] = (float)p[1].x; wh[4 * d + 1] = (float)p[3].x;
    wh[4 * d + 2] = (float)p[1].y; wh[4 * d + 3] = (float)p[3].y;
  }
}

// MXFP4: the E2M1 pairs (low nibble, high nibble) of each byte of a chunk, exact in fp32.
__device__ __forceinline__ void mxfp4_decode(uint4 w, float (&wl)[16], float (&wh)[16]) {
  const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int d = 0; d < 4; d++) {
    const v2f p0 = e2m1_pair<0>(wd[d], 1.0f), p1 = e2m1_pair<1>(wd[d], 1.0f);
    const v2f p2 = e2m1_pair<2>(wd[d], 1.0f), p3 = e2m1_pair<3>(wd[d], 1.0f);
    wl[4 * d + 0] = p0.x; wh[4 * d + 0] = p0.y;
    wl[4 * d + 1] = p1.x; wh[4 * d + 1] = p1.y;
    wl[4 * d + 2] = p2.x; wh[4 * d + 2] = p2.y;
    wl[4 * d + 3] = p3.x; wh[4 * d + 3] = p3.y;
  }
}

// sum_k w_k x_k of one chunk's decoded codes (MXFP4 before the block scale, W4A16
// before the group scale): low-nibble half, then high-nibble half, each in element
// order (the order of w4a16_chunk).
template <int HSHIFT = 0>
__device__ __forceinline__ float chunk_dot(const float (&wl)[16], const float (&wh)[16], const float4 (&xv)[8]) {
  float pl = 0.0f, ph = 0.0f;
#pragma unroll
  for (int d = 0; d < 4; d++) {
    pl = __builtin_fmaf(wl[4 * d + 0], xv[d].x, pl);
    pl = __builtin_fmaf(wl[4 * d + 1], xv[d].y, pl);
    pl = __builtin_fmaf(wl[4 * d + 2], xv[d].z, pl);
    pl = __builtin_fmaf(wl[4 * d + 3], xv[d].w, pl);
    ph = __builtin_fmaf(wh[4 * d + 0], xv[4 + d].x, ph);
    ph = __builtin_fmaf(wh[4 * d + 1], xv[4 + d].y, ph);
    ph = __builtin_fmaf(wh[4 * d + 2], xv[4 + d].z, ph);
    ph = __builtin_fmaf(wh[4 * d + 3], xv[4 + d].w, ph);
  }
  // the high half decoded at 2^HSHIFT times its value (W4A16: 16), scaled back exactly
  return HSHIFT ? pl + ph * (1.0f / (float)(1 << HSHIFT)) : pl + ph;
}

// W4A8: the exact int32 sum_k q_k a_k of one chunk (int8 dot4 on the unsigned codes,
// 0..15 being non-negative int8, against the low- and high-half activation codes).
__device__ __forceinline__ int w4a8_chunk(uint4 w, uint4 al, uint4 ah) {
  int d = 0;
  d = __builtin_amdgcn_sdot4((int)lo_nibbles(w.x), (int)al.x, d, false);
  d = __builtin_amdgcn_sdot4((int)hi_nibbles(w.x), (int)ah.x, d, false);
  d = __builtin_amdgcn_sdot4((int)lo_nibbles(w.y), (int)al.y, d, false);
  d = __builtin_amdgcn_sdot4((int)hi_nibbles(w.y), (int)ah.y, d, false);
  d = __builtin_amdgcn_sdot4((int)lo_nibbles(w.z), (int)al.z, d, false);
  d = __builtin_amdgcn_sdot4((int)hi_nibbles(w.z), (int)ah.z, d, false);
  d = __builtin_amdgcn_sdot4((int)lo_nibbles(w.w), (int)al.w, d, false);
  d = __builtin_amdgcn_sdot4((int)hi_nibbles(w.w), (int)ah.w, d, false);
  return d;
}

// acc[m][r] += this lane's share of slot r (r < nr) against activation row m (HW:
// each half-wave its own row of the slot). Chunks past the row end hold zero
// weights, zero scales and zero activations.
template <int F, int MB, int R, int NIT, bool HW>
__device__ __forceinline__ void gemv_compute(const GemvRegs<F, R, NIT> &g, float (&acc)[MB][R], int nr, int lane,
                                             int nchp, int Gp, int G, const float *xl, const uint8_t *ql,
                                             const int32_t *asl) {
  // the scale and zero-point of this lane's chunk in slot r (two rows per wave load,
  // int4: fetched from the lane holding it; lanes past the row's chunks get scale 0,
  // as their own loads past the row would have given)
  auto meta = [&](int r, int it, float &sc, int &zi) {
    if constexpr (HW && F != F_MXFP4) {
      const int ci = lane & 31, idx = (2 * r + (lane >> 5)) * G + (ci >> 2);
      const float v = __int_as_float(__builtin_amdgcn_ds_bpermute(idx * 4, __float_as_int(g.scb)));
      sc = ci < 4 * G ? v : 0.0f;
      zi = __builtin_amdgcn_ds_bpermute(idx * 4, g.zb);
    } else {
      sc = g.sc[r][it];
      zi = g.zi[r][it];
    }
  };
#pragma unroll
  for (int it = 0; it < NIT; it++) {
    const int ci = (HW ? lane & 31 : lane) + kWave * it;
    if (it * kWave >= nchp) break;  // uniform: this row length needs fewer chunks
    if constexpr (F == F_W4A16 || F == F_W4A16G32 || F == F_MXFP4) {
      // each weight row's codes decoded once, then against every activation row
#pragma unroll
      for (int r = 0; r < R; r++) {
        if (r >= nr) break;
        float wl[16], wh[16], sc;
        int zi;
        meta(r, it, sc, zi);
        if constexpr (F == F_MXFP4) {
          mxfp4_decode(g.w[r][it], wl, wh);
        } else {
          w4a16_decode(g.w[r][it], zi, wl, wh);
        }
#pragma unroll
        for (int m = 0; m < MB; m++) {
          float4 xv[8];
#pragma unroll
          for (int p = 0; p < 8; p++)
            xv[p] = *reinterpret_cast<const float4 *>(xl + ((size_t)(m * 8 + p) * nchp + ci) * 4);
          const float part = F == F_MXFP4 ? chunk_dot(wl, wh, xv) : chunk_dot<4>(wl, wh, xv);
          acc[m][r] = __builtin_fmaf(sc, part, acc[m][r]);
        }
      }
    } else {
      // W4A8: the group's zero-point term z * sum(a) is taken once, by the lane
      // holding the group's first 16 bytes. Each lane's integer is exact and below
      // 2^24, so its conversion to fp32 is exact.
      const int gi = fmt_g32(F) ? ci : ci >> 2;
      const bool first = fmt_g32(F) || (ci & 3) == 0;
#pragma unroll
      for (int m = 0; m < MB; m++) {
        const uint4 al = *reinterpret_cast<const uint4 *>(ql + ((size_t)(m * 2 + 0) * nchp + ci) * 16);
        const uint4 ah = *reinterpret_cast<const uint4 *>(ql + ((size_t)(m * 2 + 1) * nchp + ci) * 16);
        const int as = first ? asl[m * Gp + gi] : 0;
#pragma unroll
        for (int r = 0; r < R; r++) {
          if (r >= nr) break;
          float sc;
          int zi;
          meta(r, it, sc, zi);
          int d = w4a8_chunk(g.w[r][it], al, ah);
          d -= zi * as;
          acc[m][r] = __builtin_fmaf(sc, (float)d, acc[m][r]);
        }
      }
    }
  }
}

// The persistent grid puts two 8-wave workgroups on every CU, i.e. four waves per
// SIMD, which needs at most 128 VGPRs per lane; the int8 one-row kernels without a
// prologue are asked to fit (their longest-row variants would otherwise use a few
// more, and the second workgroup of every CU would wait for the first). The fp32
// kernels of rows past 8192 elements, and the prologue variants, need far more and
// are left unconstrained.
template <int F, int MB, int PRO>
struct GemvMinWaves {
  static constexpr int value = (F == F_W4A8 || F == F_W4A8G32) && MB == 1 && PRO == 0 ? 4 : 1;
};

// PRO selects a fused prologue on the (single, register-held) activation row:
// 0 none, 1 RMSNorm (x * (1 / sqrt(mean(x^2) + eps)) * norm_w, the mean over Kp),
// 2 SwiGLU (the row is [gate | up], Kp floats each: silu(gate) * up), 3 attention
// merge (the row is merged from one-token attention partials, attn_merge8: every
// thread's partials are requested before the weights, rows up to 2048). The epilogue
// adds `bias` and `res` when given and max-combines argmax keys into `amax_key`;
// under `glu` it writes silu(gate) * up of each (gate, up) row pair instead.
// HW (rows of at most 1024 elements, one activation row): every wave load covers
// two weight rows, one per half-wave, so no lane idles past a short row's end.
template <int F, int MB, int R, int NIT, int PRO, bool HW = false>
__global__ __launch_bounds__(kGemvThreads) __attribute__((amdgpu_waves_per_eu(GemvMinWaves<F, MB, PRO>::value)))
void gemv_kernel(GemmArgs a) {
  static_assert(!HW || (MB == 1 && NIT == 1), "two rows per wave load: one activation row, one chunk per lane");
  constexpr int RR = HW ? 2 * R : R;  // weight rows per batch (R slots)
  extern __shared__ __align__(16) unsigned char lds[];
  __shared__ float red[2][kGemvWaves];
  constexpr bool kInt8 = (F == F_W4A8 || F == F_W4A8Q || F == F_W4A8G32);
  constexpr int T = kGemvThreads;
  const int Kp = a.Kp, N = a.N;
  const int nch = Kp >> 5;                        // 16-byte chunks per weight row
  const int nit = (nch + kWave - 1) / kWave;      // <= NIT
  const int nchp = nit * kWave;                   // plane entries (padded)
  // groups per row, and per row of the LDS group sums (padded like the planes)
  const int G = Kp / fmt_group(F), Gp = fmt_g32(F) ? nchp : nchp / 4;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int gw = blockIdx.x * kGemvWaves + wave, W = gridDim.x * kGemvWaves;
  // wave gw takes rows [r0, r1): NU / W units of u rows each (u = 2 under the glu
  // epilogue, whose gate/up pairs must share a wave), one more for the first NU % W waves
  const int u = a.glu ? 2 : 1, NU = a.glu ? N >> 1 : N;
  const int ubase = (int)((unsigned)NU / (unsigned)W), urem = NU - ubase * W;
  const int r0 = u * (gw * ubase + min(gw, urem)), r1 = r0 + u * (ubase + (gw < urem ? 1 : 0));

  float *xl = reinterpret_cast<float *>(lds);                           // fp32 planes [MB][8][nchp][4]
  uint8_t *ql = lds;                                                      // int8 planes [MB][2][nchp][16]
  int32_t *asl = reinterpret_cast<int32_t *>(lds + (size_t)MB * nchp * 32);  // [MB][Gp]
  float *xsl = reinterpret_cast<float *>(asl + (size_t)MB * Gp);         // [MB]

  // ---- 1. activations into registers, issued first: NIT float4 per thread per
  //         row (slots past Kp read 0 through the row's buffer descriptor)
  constexpr int S = NIT;
  constexpr bool kXReg = (F != F_W4A8Q) && MB * S <= kXRegs;
  static_assert(PRO == 0 || (MB == 1 && kXReg), "prologues take one register-held activation row");
  float4 xr[kXReg ? MB * S : 1];
  float4 xe[(PRO == 1 || PRO == 2) ? S : 1];  // RMSNorm weights, or the up half of a SwiGLU row
  static_assert(PRO != 3 || S == 1, "the attention-merge prologue takes rows up to 2048 elements");
  AttnPart8 apt[1];  // attention merge: the partials of this thread's float4
  if constexpr (PRO == 3) {
    // this thread's float4 belongs to head e / D: all its slices' partials
    const int e = threadIdx.x * 4, D = a.attn_d, PS = D + 4;
    if (e < Kp) attn_fetch8(apt[0], a.attn_part + (size_t)(e / D) * a.attn_ns * PS, PS, D, 0, a.attn_ns, (e % D) / 4);
  } else if constexpr (kXReg) {
#pragma unroll
    for (int m = 0; m < MB; m++) {
      const Rsrc rx = make_rsrc(a.x + (size_t)m * Kp, (uint32_t)Kp * 4);
#pragma unroll
      for (int i = 0; i < S; i++) xr[m * S + i] = ld_f4(rx, (threadIdx.x + i * T) * 16);
    }
    if constexpr (PRO != 0) {
      const Rsrc re = make_rsrc(PRO == 1 ? a.norm_w : a.x + Kp, (uint32_t)Kp * 4);
#pragma unroll
      for (int i = 0; i < S; i++) xe[i] = ld_f4(re, (threadIdx.x + i * T) * 16);
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // keep the activation loads ahead of the weight stream

  // ---- 2. the weight stream of this wave's first R rows, then their epilogue
  //         operands (bias, residual), so that the epilogue waits for no load
  //         (the epilogue runs once per window of up to WN rows, one row per lane:
  //         lane j's operands are those of row wb + j)
  GemvRegs<F, R, NIT> g;
  float bv = 0.0f, rv[MB];
  auto epi_load = [&](int wb) {
    const int n = wb + lane < N ? wb + lane : N - 1;  // rows past the share are never stored
    if (a.bias) bv = a.bias[n];
#pragma unroll
    for (int m = 0; m < MB; m++) rv[m] = a.res ? a.res[(size_t)m * N + n] : 0.0f;
  };
  epi_load(r0);  // ahead of the weights: a wait for the weights then covers these too
  gemv_load<F, R, NIT, HW>(a, g, r0, r1, lane, nch, G);
  __builtin_amdgcn_sched_barrier(0);

  // ---- 3. fused prologue, then stage the activations into LDS while the weights
  //         are in flight (slot i covers elements [2048 i, 2048 i + 2048); slots
  //         past the padded plane length are skipped on a block-uniform branch;
  //         elements past Kp are 0 and stay 0 under both prologues)
  if constexpr (PRO == 1) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < S; i++) {
      ss = __builtin_fmaf(xr[i].x, xr[i].x, ss);
      ss = __builtin_fmaf(xr[i].y, xr[i].y, ss);
      ss = __builtin_fmaf(xr[i].z, xr[i].z, ss);
      ss = __builtin_fmaf(xr[i].w, xr[i].w, ss);
    }
    ss = wave_sum(ss);
    // red[1]: the one-row quantizer below uses red[0] only, so no second barrier
    // is needed before it overwrites anything
    if (lane == 0) red[1][wave] = ss;
    __syncthreads();
    float tot = red[1][0];
#pragma unroll
    for (int w = 1; w < kGemvWaves; w++) tot += red[1][w];
    const float rn = 1.0f / sqrtf(tot / (float)Kp + a.norm_eps);
#pragma unroll
    for (int i = 0; i < S; i++) {
      xr[i].x = xr[i].x * rn * xe[i].x;
      xr[i].y = xr[i].y * rn * xe[i].y;
      xr[i].z = xr[i].z * rn * xe[i].z;
      xr[i].w = xr[i].w * rn * xe[i].w;
    }
  } else if constexpr (PRO == 3) {
    xr[0] = (int)threadIdx.x * 4 < Kp ? attn_merge8(apt[0], a.attn_ns) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  } else if constexpr (PRO == 2) {
#pragma unroll
    for (int i = 0; i < S; i++) {
      xr[i].x = xr[i].x / (1.0f + expf(-xr[i].x)) * xe[i].x;
      xr[i].y = xr[i].y / (1.0f + expf(-xr[i].y)) * xe[i].y;
      xr[i].z = xr[i].z / (1.0f + expf(-xr[i].z)) * xe[i].z;
      xr[i].w = xr[i].w / (1.0f + expf(-xr[i].w)) * xe[i].w;
    }
  }
  if constexpr (!kInt8) {
    if constexpr (kXReg) {
#pragma unroll
      for (int j = 0; j < MB * S; j++) {
        const int m = j / S, i = j % S;
        if (i >= nit) continue;
        int ci, half, within;
        chunk_pos(F, threadIdx.x * 4 + i * T * 4, ci, half, within);
        *reinterpret_cast<float4 *>(xl + ((size_t)(m * 8 + half * 4 + (within >> 2)) * nchp + ci) * 4) = xr[j];
      }
    } else {
      for (int m = 0; m < MB; m++) {
        const Rsrc rx = make_rsrc(a.x + (size_t)m * Kp, (uint32_t)Kp * 4);
        for (int e = threadIdx.x * 4; e < nchp * 32; e += T * 4) {
          int ci, half, within;
          chunk_pos(F, e, ci, half, within);
          *reinterpret_cast<float4 *>(xl + ((size_t)(m * 8 + half * 4 + (within >> 2)) * nchp + ci) * 4) =
              ld_f4(rx, e * 4);
        }
      }
    }
  } else if constexpr (F == F_W4A8 || F == F_W4A8G32) {
    // fused per-token quantizer: bit-identical to quant_rows_kernel (unrolled over
    // the rows, so that xr is indexed by constants and stays in registers)
#pragma unroll
    for (int m = 0; m < MB; m++) {
      const Rsrc rx = make_rsrc(a.x + (size_t)m * Kp, (uint32_t)Kp * 4);
      float amax = 0.0f;  // padding reads +0 and cannot raise it
      if constexpr (kXReg) {
#pragma unroll
        for (int i = 0; i < S; i++) {
          const float4 v = xr[m * S + i];
          amax = fmaxf(fmaxf(amax, fabsf(v.x)), fabsf(v.y));
          amax = fmaxf(fmaxf(amax, fabsf(v.z)), fabsf(v.w));
        }
      } else {
        for (int e = threadIdx.x * 4; e < Kp; e += T * 4) {
          const float4 v = ld_f4(rx, e * 4);
          amax = fmaxf(fmaxf(amax, fabsf(v.x)), fabsf(v.y));
          amax = fmaxf(fmaxf(amax, fabsf(v.z)), fabsf(v.w));
        }
      }
      // red[m & 1]: row m + 1 writes the other half, and row m + 2 comes after
      // row m + 1's barrier, by which time every wave has read row m's partials
      amax = wave_max(amax);
      if (lane == 0) red[m & 1][wave] = amax;
      __syncthreads();
      float rmax = red[m & 1][0];
#pragma unroll
      for (int w = 1; w < kGemvWaves; w++) rmax = fmaxf(rmax, red[m & 1][w]);
      const float sc = row_scale(rmax);
      const float inv = 1.0f / sc;
      if (threadIdx.x == 0) xsl[m] = sc;
      // thread t quantizes 4 elements per slot; a group of 128 is one half-wave
      for (int i = 0; i < nit; i++) {
        const int e = threadIdx.x * 4 + i * T * 4;
        float4 v;
        if constexpr (kXReg) {
          v = xr[m * S];
#pragma unroll
          for (int k = 1; k < S; k++)
            if (k == i) v = xr[m * S + k];
        } else {
          v = ld_f4(rx, e * 4);
        }
        int ci, half, within;
        chunk_pos(F, e, ci, half, within);
        const uint32_t qv = quant4_fast(v, sc, inv);
        *reinterpret_cast<uint32_t *>(ql + ((size_t)(m * 2 + half) * nchp + ci) * 16 + within) = qv;
        if constexpr (F == F_W4A8G32) {
          // a group of 32 is eight threads
          const int gs = eighth_wave_sum(sum_i8x4(qv));
          if ((threadIdx.x & 7) == 7) asl[m * Gp + (e >> 5)] = gs;
        } else {
          const int gs = half_wave_sum(sum_i8x4(qv));
          if ((threadIdx.x & 31) == 31) asl[m * Gp + (e >> 7)] = gs;
        }
      }
    }
  } else {
    for (int m = 0; m < MB; m++) {
      const Rsrc rq = make_rsrc(a.xq + (size_t)m * Kp, (uint32_t)Kp);
      for (int e = threadIdx.x * 4; e < nchp * 32; e += T * 4) {
        int ci, half, within;
        chunk_pos(F, e, ci, half, within);
        *reinterpret_cast<uint32_t *>(ql + ((size_t)(m * 2 + half) * nchp + ci) * 16 + within) = ld_u32(rq, e);
      }
      for (int gg = threadIdx.x; gg < Gp; gg += T) asl[m * Gp + gg] = gg < G ? a.asum[(size_t)m * G + gg] : 0;
      if (threadIdx.x == 0) xsl[m] = a.xs[m];
    }
  }
  __syncthreads();

  // ---- 4. decode + accumulate R rows at a time; later batches load as the
  //         previous one finishes. Each row's total goes to lane (row - wb) of
  //         `sum` for a window of WN rows starting at wb (a whole number of batches,
  //         even, so that glu pairs never straddle windows); the epilogue then runs
  //         once per window with one row per lane and one coalesced store.
  constexpr int WN = (RR & 1) ? (kWave / (2 * RR)) * (2 * RR) : (kWave / RR) * RR;
  unsigned long long best = 0;  // this lane's argmax key over the wave's windows
  float sum[MB];
  for (int wb = r0; wb < r1; wb += WN) {
    const int we = min(wb + WN, r1);
    if (wb != r0) epi_load(wb);
#pragma unroll
    for (int m = 0; m < MB; m++) sum[m] = 0.0f;
    for (int rb = wb; rb < we; rb += RR) {
      if (rb != r0) gemv_load<F, R, NIT, HW>(a, g, rb, r1, lane, nch, G);
      const int nr = min(RR, r1 - rb);          // rows of this batch
      const int ns = HW ? (nr + 1) >> 1 : nr;   // slots holding them
      float acc[MB][R];
#pragma unroll
      for (int m = 0; m < MB; m++)
#pragma unroll
        for (int r = 0; r < R; r++) acc[m][r] = 0.0f;
      gemv_compute<F, MB, R, NIT, HW>(g, acc, ns, lane, nchp, Gp, G, xl, ql, asl);
      // ---- 5. one wave (HW: half-wave) reduction per output, into its lane of `sum`
#pragma unroll
      for (int m = 0; m < MB; m++) {
#pragma unroll
        for (int r = 0; r < R; r++) {
          if (r >= ns) break;
          if constexpr (HW) {
            const float v = half_wave_sum_f(acc[m][r]);
            const int j = rb + 2 * r - wb;
            write_lane(sum[m], __builtin_amdgcn_readlane(__float_as_int(v), 31), j);
            write_lane(sum[m], __builtin_amdgcn_readlane(__float_as_int(v), 63), j + 1);
          } else {
            write_lane(sum[m], __float_as_int(wave_sum(acc[m][r])), rb + r - wb);
          }
        }
      }
    }
    // ---- 6. the window's epilogue: lane j holds row n = wb + j
    const int n = wb + lane;
    const bool live = n < we;
#pragma unroll
    for (int m = 0; m < MB; m++) {
      float t = sum[m];
      {
        // y is rounded before the bias and the residual are added, as separate
        // float32 adds after the GEMM would round it (no fused multiply-add)
#pragma clang fp contract(off)
        if constexpr (kInt8) t *= xsl[m];
        if (a.bias) t += bv;
        if (a.res) t = rv[m] + t;
      }
      if (a.glu) {
        // wb is even, so even lanes hold gates and the next lane their up row
        const float up = dpp_f<kDppQuad1032>(t, 0.0f);
        t = t / (1.0f + expf(-t)) * up;  // the SwiGLU kernel's expression
        if (live && (lane & 1) == 0) a.y[(size_t)m * (N >> 1) + (n >> 1)] = t;
      } else {
        if (live) a.y[(size_t)m * N + n] = t;
        if (a.amax_key && live) {
          const unsigned long long k = argmax_key(t, n);
          best = k > best ? k : best;
        }
      }
    }
  }
  // spread over the slots so that no address takes more than a few atomics
  if (a.amax_key) {
    best = wave_max_u64(best);
    if (lane == 0 && best) atomicMax(a.amax_key + gw % kArgmaxSlots, best);
  }
}

using GemvFn = void (*)(GemmArgs);

// ============================================================ paced decode GEMV (M = 1)
//
// The plain decode GEMV (one activation row, no fused prologue or epilogue) on rows
// of more than 1024 elements. A CU accepts only a limited number of outstanding
// vector-memory instructions: a wave that issues all its weight loads up front stalls
// at the issue of the later ones until the queue drains, and everything behind them
// in program order (the activation prologue, then the compute) waits too, so compute
// ran only after most of the stream had arrived. Here each wave issues the loads of
// one row, runs the prologue (activations staged in LDS; for W4A8 the per-token
// quantizer), then per row issues the next row's loads before it waits for and
// computes the current one (two register stages, the next row always in flight).
// Loads are unconditional (rows past the wave's share read zero-length ranges), so
// every wait counts exactly the loads it needs. Weight, scale, zero-point and E8M0
// loads are non-temporal: each byte is read once per call.
//
// The per-lane arithmetic and the wave reduction are those of gemv_kernel
// (gemv_compute), so the outputs equal that kernel's bit for bit.

constexpr int kPacedAux = kWeightAux;  // the weight and metadata loads: non-temporal

// One weight row in flight: NIT 16-byte chunks per lane and, per chunk, the raw scale
// bits (int4: fp32 of the chunk's group; MXFP4: the E8M0 byte of its block) and the
// zero-point byte (int4); bytes are converted where they are used.
template <int NIT>
struct PacedStage {
  uint4 w[NIT];
  uint32_t s[NIT];
  uint32_t z[NIT];
};

// DW: the zero-point (int4) and E8M0 (MXFP4) bytes come as the aligned dword that
// holds them, extracted where they are used. A byte load's value carried across the
// row loop is masked at the loop edge, which waits for the whole stage and stalls the
// next row's issue; dword values are carried as they are. Taken where every row's
// bytes fill whole dwords (G or the block count a multiple of 4), so no dword reaches
// past a row: every byte is in bounds.
template <int F, int NIT, bool DW>
__device__ __forceinline__ void paced_load(const GemmArgs &a, PacedStage<NIT> &st, int row, int r1, int lane,
                                           int nch, int G, uint32_t cbase = 0) {
  const uint32_t rowbytes = (uint32_t)(a.Kp >> 1);
  const bool in = row < r1;
  const size_t rr = in ? (size_t)row : 0;
  const Rsrc rw = make_rsrc(a.qw + rr * rowbytes, in ? rowbytes : 0u);
  if constexpr (F == F_MXFP4) {
    const Rsrc re = make_rsrc(a.e8m0 + rr * nch, in ? (uint32_t)nch : 0u);
#pragma unroll
    for (int it = 0; it < NIT; it++) {
      const uint32_t ci = cbase + (uint32_t)lane + kWave * it;
      const v4u v = __builtin_amdgcn_raw_buffer_load_b128(rw, (int)(ci * 16), 0, kPacedAux);
      st.w[it] = make_uint4(v.x, v.y, v.z, v.w);
      if constexpr (DW) st.s[it] = __builtin_amdgcn_raw_buffer_load_b32(re, (int)(ci & ~3u), 0, kPacedAux);
      else st.s[it] = __builtin_amdgcn_raw_buffer_load_b8(re, (int)ci, 0, kPacedAux);
      st.z[it] = 0;
      __builtin_amdgcn_sched_barrier(0);  // a chunk's loads together: its compute waits for them alone
    }
  } else {
    const Rsrc rs = make_rsrc(a.scales + rr * G, in ? (uint32_t)G * 4 : 0u);
    const Rsrc rz = make_rsrc(a.zeros ? a.zeros + rr * G : a.qw, (in && a.zeros) ? (uint32_t)G : 0u);
    auto gidx = [&](int it) {
      const uint32_t ci = cbase + (uint32_t)lane + kWave * it;
      return fmt_g32(F) ? ci : ci >> 2;
    };
    auto zload = [&](int it) {
      if constexpr (DW) st.z[it] = __builtin_amdgcn_raw_buffer_load_b32(rz, (int)(gidx(it) & ~3u), 0, kPacedAux);
      else st.z[it] = __builtin_amdgcn_raw_buffer_load_b8(rz, (int)gidx(it), 0, kPacedAux);
    };
    if constexpr (F == F_W4A16 || F == F_W4A16G32) {
      // loads return in issue order, and W4A16 needs every chunk's zero-point before
      // its products (q - z) and the scales after them: the zero-points first, then
      // the weights chunk by chunk, then the scales
#pragma unroll
      for (int it = 0; it < NIT; it++) zload(it);
#pragma unroll
      for (int it = 0; it < NIT; it++) {
        const v4u v = __builtin_amdgcn_raw_buffer_load_b128(rw, (int)((cbase + lane + kWave * it) * 16), 0, kPacedAux);
        st.w[it] = make_uint4(v.x, v.y, v.z, v.w);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int it = 0; it < NIT; it++) st.s[it] = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)(gidx(it) * 4), 0, kPacedAux);
      __builtin_amdgcn_sched_barrier(0);
    } else {
#pragma unroll
      for (int it = 0; it < NIT; it++) {
        const uint32_t ci = cbase + (uint32_t)lane + kWave * it;
        const v4u v = __builtin_amdgcn_raw_buffer_load_b128(rw, (int)(ci * 16), 0, kPacedAux);
        st.w[it] = make_uint4(v.x, v.y, v.z, v.w);
        st.s[it] = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)(gidx(it) * 4), 0, kPacedAux);
        zload(it);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
}

// The byte of chunk `ci` in a stage's metadata word (DW: the dword holding it).
template <int F, bool DW>
__device__ __forceinline__ uint32_t paced_byte(uint32_t word, uint32_t ci) {
  if constexpr (!DW) return word & 0xFFu;
  const uint32_t idx = fmt_group(F) == 32 ? ci : ci >> 2;  // block or group index
  return (word >> (8 * (idx & 3u))) & 0xFFu;
}

template <int F, int NIT, bool DW>
__global__ __launch_bounds__(kGemvThreads) void gemv_paced_kernel(GemmArgs a) {
  constexpr bool kInt8 = (F == F_W4A8 || F == F_W4A8Q || F == F_W4A8G32);
  constexpr bool kW16 = (F == F_W4A16 || F == F_W4A16G32);  // int4 codes, fp32 activations
  constexpr int T = kGemvThreads;
  extern __shared__ __align__(16) unsigned char lds[];
  __shared__ float red[kGemvWaves];
  const int Kp = a.Kp;
  const int nch = Kp >> 5;
  const int nit = (nch + kWave - 1) / kWave;
  const int nchp = nit * kWave;
  const int G = Kp / fmt_group(F), Gp = fmt_g32(F) ? nchp : nchp / 4;  // padded group count
  // ---- 1. the activation row into registers (the kernel's first loads), then the
  //         row shares and the first row's weights
  constexpr int S = NIT;
  float4 xr[F == F_W4A8Q ? 1 : S];
  if constexpr (F != F_W4A8Q) {
    const Rsrc rx = make_rsrc(a.x, (uint32_t)Kp * 4);
#pragma unroll
    for (int i = 0; i < S; i++) xr[i] = ld_f4(rx, (threadIdx.x + i * T) * 16);
  }
  __builtin_amdgcn_sched_barrier(0);
  // W4A8 and W4A16: about 256 clocks between the activation loads and the first
  // weight loads, so that the activations, whose prologue (the int8 quantizer, the
  // W4A16 chunk sums) gates every row, queue ahead of the weight stream (1 x 11008 x
  // 4096 cold: W4A8 6.23 -> 5.77 us, W4A16 6.49 -> 6.40; 64 and 128 clocks gain
  // less, 320 and more lose again; MXFP4 gains nothing)
  if constexpr (F == F_W4A8 || F == F_W4A8G32 || kW16) __builtin_amdgcn_s_sleep(4);
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  // rows of this workgroup (an even share: N / grid and N % grid come from the host),
  // then of this wave; the empty asm keeps the scalar work of the split behind the
  // activation loads (the instruction selector would otherwise place it first)
  unsigned bx = blockIdx.x;
  asm volatile("" : "+s"(bx));
  const unsigned base = (unsigned)a.split_base, rem = (unsigned)a.split_rem;
  const int wr0 = (int)(bx * base + min(bx, rem)), wn = (int)(base + (bx < rem ? 1u : 0u));
  const int r0 = wr0 + (wave * wn) / kGemvWaves, r1 = wr0 + ((wave + 1) * wn) / kGemvWaves;

  float *xl = reinterpret_cast<float *>(lds);
  uint8_t *ql = lds;
  int32_t *asl = reinterpret_cast<int32_t *>(lds + (size_t)nchp * 32);
  float *xsl = reinterpret_cast<float *>(asl + Gp);
  PacedStage<NIT> st0, st1;
  paced_load<F, NIT, DW>(a, st0, r0, r1, lane, nch, G);
  __builtin_amdgcn_sched_barrier(0);

  // ---- 2. the prologue: stage (or quantize) the activations into the LDS planes
  if constexpr (kW16 || F == F_MXFP4) {
#pragma unroll
    for (int i = 0; i < S; i++) {
      if (i >= nit) continue;
      int ci, half, within;
      chunk_pos(F, threadIdx.x * 4 + i * T * 4, ci, half, within);
      *reinterpret_cast<float4 *>(xl + ((size_t)(half * 4 + (within >> 2)) * nchp + ci) * 4) = xr[i];
    }
  } else if constexpr (F == F_W4A8 || F == F_W4A8G32) {
    float amax = 0.0f;  // padding reads +0 and cannot raise it
#pragma unroll
    for (int i = 0; i < S; i++) {
      amax = fmaxf(fmaxf(amax, fabsf(xr[i].x)), fabsf(xr[i].y));
      amax = fmaxf(fmaxf(amax, fabsf(xr[i].z)), fabsf(xr[i].w));
    }
    amax = wave_max(amax);
    if (lane == 0) red[wave] = amax;
    __syncthreads();
    float rmax = red[0];
#pragma unroll
    for (int w = 1; w < kGemvWaves; w++) rmax = fmaxf(rmax, red[w]);
    const float sc = rmax > 0.0f ? div127(rmax) : 1.0f;  // row_scale, bit for bit
    const float inv = 1.0f / sc;
    if (threadIdx.x == 0) xsl[0] = sc;
#pragma unroll
    for (int i = 0; i < S; i++) {
      if (i >= nit) continue;
      const int e = threadIdx.x * 4 + i * T * 4;
      int ci, half, within;
      chunk_pos(F, e, ci, half, within);
      const uint32_t qv = quant4_fast(xr[i], sc, inv);
      *reinterpret_cast<uint32_t *>(ql + ((size_t)half * nchp + ci) * 16 + within) = qv;
      if constexpr (F == F_W4A8G32) {
        const int gs = eighth_wave_sum(sum_i8x4(qv));  // a group of 32 is eight threads
        if ((threadIdx.x & 7) == 7) asl[e >> 5] = gs;
      } else {
        const int gs = half_wave_sum(sum_i8x4(qv));  // a group of 128 is one half-wave
        if ((threadIdx.x & 31) == 31) asl[e >> 7] = gs;
      }
    }
  } else {  // F_W4A8Q: codes, group sums and the token scale as given
    const Rsrc rq = make_rsrc(a.xq, (uint32_t)Kp);
    for (int e = threadIdx.x * 4; e < nchp * 32; e += T * 4) {
      int ci, half, within;
      chunk_pos(F, e, ci, half, within);
      *reinterpret_cast<uint32_t *>(ql + ((size_t)half * nchp + ci) * 16 + within) = ld_u32(rq, e);
    }
    for (int gg = threadIdx.x; gg < Gp; gg += T) asl[gg] = gg < G ? a.asum[gg] : 0;
    if (threadIdx.x == 0) xsl[0] = a.xs[0];
  }
  __syncthreads();

  // ---- 3. this lane's activation operands into registers (rows up to 4096 elements:
  //         fp32, 64 VGPRs, or int8 codes, 16), read from the LDS planes once
  constexpr bool kXReg = NIT <= 2;
  constexpr bool kF32 = (kW16 || F == F_MXFP4);
  float4 xv[kXReg && kF32 ? NIT : 1][8];
  uint4 al[kXReg && kInt8 ? NIT : 1], ah[kXReg && kInt8 ? NIT : 1];
  int as[kXReg && kInt8 ? NIT : 1];
  if constexpr (kXReg) {
#pragma unroll
    for (int it = 0; it < NIT; it++) {
      const int ci = lane + kWave * it;  // NIT == nit: the planes hold every chunk
      if constexpr (kF32) {
#pragma unroll
        for (int p = 0; p < 8; p++) xv[it][p] = *reinterpret_cast<const float4 *>(xl + ((size_t)p * nchp + ci) * 4);
      } else {
        al[it] = *reinterpret_cast<const uint4 *>(ql + (size_t)ci * 16);
        ah[it] = *reinterpret_cast<const uint4 *>(ql + ((size_t)nchp + ci) * 16);
        // the zero-point term once per group, by the lane holding its first chunk
        if constexpr (fmt_g32(F)) as[it] = asl[ci];
        else as[it] = (ci & 3) == 0 ? asl[ci >> 2] : 0;
      }
    }
  }

  // ---- 4. rows: the next one's loads out, then this one's compute, reduction and store
  const int zadd = a.zeros ? 0 : 8;
  const float xs = kInt8 ? xsl[0] : 1.0f;  // the token scale (W4A8)
  auto row_out = [&](const PacedStage<NIT> &st, int row) {
    float acc = 0.0f;
    if constexpr (kXReg) {
#pragma unroll
      for (int it = 0; it < NIT; it++) {
        const uint32_t ci = (uint32_t)lane + kWave * it;
        if constexpr (kW16) {
          const int z = (int)paced_byte<F, DW>(st.z[it], ci) + zadd;
          acc = __builtin_fmaf(__uint_as_float(st.s[it]), w4a16_chunk(st.w[it], xv[it], z), acc);
        } else if constexpr (F == F_MXFP4) {
          float wl[16], wh[16];
          mxfp4_decode(st.w[it], wl, wh);
          acc = __builtin_fmaf(e8m0_to_f32(paced_byte<F, DW>(st.s[it], ci)), chunk_dot(wl, wh, xv[it]), acc);
        } else {
          int d = w4a8_chunk(st.w[it], al[it], ah[it]);
          d -= ((int)paced_byte<F, DW>(st.z[it], ci) + zadd) * as[it];
          acc = __builtin_fmaf(__uint_as_float(st.s[it]), (float)d, acc);
        }
      }
    } else {
      GemvRegs<F, 1, NIT> g;
#pragma unroll
      for (int it = 0; it < NIT; it++) {
        const uint32_t ci = (uint32_t)lane + kWave * it;
        g.w[0][it] = st.w[it];
        if constexpr (F == F_MXFP4) {
          g.sc[0][it] = e8m0_to_f32(paced_byte<F, DW>(st.s[it], ci));
          g.zi[0][it] = 0;
        } else {
          g.sc[0][it] = __uint_as_float(st.s[it]);
          g.zi[0][it] = (int)paced_byte<F, DW>(st.z[it], ci) + zadd;
        }
      }
      float ac[1][1] = {{0.0f}};
      gemv_compute<F, 1, 1, NIT, false>(g, ac, 1, lane, nchp, Gp, G, xl, ql, asl);
      acc = ac[0][0];
    }
    float t = wave_sum(acc);
    if constexpr (kInt8) {
#pragma clang fp contract(off)
      t *= xs;
    }
    if (lane == 0) a.y[row] = t;
  };
  // steady state: two rows per iteration, the next row always in flight (stage 0 holds
  // row r on entry); then the last one or two rows, whose loads are all out already
  int r = r0;
  for (; r + 2 < r1; r += 2) {
    paced_load<F, NIT, DW>(a, st1, r + 1, r1, lane, nch, G);
    __builtin_amdgcn_sched_barrier(0);
    row_out(st0, r);
    __builtin_amdgcn_sched_barrier(0);
    paced_load<F, NIT, DW>(a, st0, r + 2, r1, lane, nch, G);
    __builtin_amdgcn_sched_barrier(0);
    row_out(st1, r + 1);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (r + 1 < r1) {
    paced_load<F, NIT, DW>(a, st1, r + 1, r1, lane, nch, G);
    __builtin_amdgcn_sched_barrier(0);
    row_out(st0, r);
    __builtin_amdgcn_sched_barrier(0);
    row_out(st1, r + 1);
  } else if (r < r1) {
    row_out(st0, r);
  }
}

// ============================================================ paced decode GEMV, rows split (M = 1, K > 4096)
//
// W4A16 (either group size) and MXFP4 rows of more than 128 chunks (4096 elements): their fp32
// activations no longer fit a wave's registers (64 VGPRs hold two chunks per lane),
// and reading them from LDS for every row costs more LDS bandwidth than the row's
// weights (4096 x 11008: 44 KB per row, 16 waves per CU). Here a row's chunks are cut
// into S slices of 128 chunks (two per lane). Wave w of a workgroup takes slice w % S,
// the waves of one slice split the workgroup's rows evenly, and each wave holds its
// slice's activations in registers for all its rows: LDS serves 16 KB per wave once.
// Per row a wave sums its slice as the one-row kernel sums a row (same per-chunk
// helpers, same two stages in flight); the slices' sums meet in LDS, and after one
// barrier the workgroup adds them in slice order and stores the row. The activation
// planes are padded to S * 128 chunks (zeros), so a slice past the row's end adds
// exactly 0. (W4A8, whose int8 codes cost a quarter of the LDS bytes, measured no
// faster this way: 8.48 -> 8.42 us cold, 7.51 -> 7.80 us hot at 1 x 4096 x 11008.)
// WV waves per workgroup (a multiple of S where it matters: every slice then gets
// as many waves as the others); SMAX the most slices the instantiation stages.
constexpr int kSplitChunks = 2 * kWave;  // chunks per slice

template <int F, bool DW, int WV = kGemvWaves, int SMAX = 4>
__global__ __launch_bounds__(WV * kWave) void gemv_paced_split_kernel(GemmArgs a) {
  static_assert(F == F_W4A16 || F == F_W4A16G32 || F == F_MXFP4, "fp32 activations");
  constexpr bool kW16 = (F == F_W4A16 || F == F_W4A16G32);
  // X staging: the float4 of up to SMAX slices over the workgroup's threads
  constexpr int T = WV * kWave, NIT = 2, SX = (SMAX * kSplitChunks * 8 + T - 1) / T;
  extern __shared__ __align__(16) unsigned char lds[];
  const int Kp = a.Kp;
  const int nch = Kp >> 5;
  const int S = (nch + kSplitChunks - 1) / kSplitChunks;  // 2..4 (the host checks)
  const int nchp = S * kSplitChunks;                      // plane entries, whole slices
  const int G = Kp / fmt_group(F);
  // ---- 1. the activation row (whole slices; slots past Kp read 0), the kernel's
  //         first loads
  float4 xr[SX];
  {
    const Rsrc rx = make_rsrc(a.x, (uint32_t)Kp * 4);
#pragma unroll
    for (int i = 0; i < SX; i++) xr[i] = ld_f4(rx, (threadIdx.x + i * T) * 16);
  }
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (kW16) __builtin_amdgcn_s_sleep(4);  // as in the one-row kernel
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  unsigned bx = blockIdx.x;
  asm volatile("" : "+s"(bx));
  const unsigned base = (unsigned)a.split_base, rem = (unsigned)a.split_rem;
  const int wr0 = (int)(bx * base + min(bx, rem)), wn = (int)(base + (bx < rem ? 1u : 0u));
  // slice sl of this wave, its index j among the P waves of that slice, its rows
  const int sl = wave % S, j = wave / S, P = (WV - 1 - sl) / S + 1;
  const int r0 = wr0 + (j * wn) / P, r1 = wr0 + ((j + 1) * wn) / P;
  const uint32_t cb = (uint32_t)sl * kSplitChunks;

  float *xl = reinterpret_cast<float *>(lds);
  float *part = xl + (size_t)nchp * 32;  // the slices' row sums, [row of the workgroup][slice]
  PacedStage<NIT> st0, st1;
  paced_load<F, NIT, DW>(a, st0, r0, r1, lane, nch, G, cb);
  __builtin_amdgcn_sched_barrier(0);

  // ---- 2. stage the activations of all S slices into the LDS planes
#pragma unroll
  for (int i = 0; i < SX; i++) {
    if ((int)threadIdx.x + i * T >= S * kSplitChunks * 8) continue;  // past the S slices' float4
    int ci, half, within;
    chunk_pos(F, threadIdx.x * 4 + i * T * 4, ci, half, within);
    *reinterpret_cast<float4 *>(xl + ((size_t)(half * 4 + (within >> 2)) * nchp + ci) * 4) = xr[i];
  }
  __syncthreads();

  // ---- 3. this wave's slice of the activations into registers
  float4 xv[NIT][8];
#pragma unroll
  for (int it = 0; it < NIT; it++) {
    const int ci = (int)cb + lane + kWave * it;
#pragma unroll
    for (int p = 0; p < 8; p++) xv[it][p] = *reinterpret_cast<const float4 *>(xl + ((size_t)p * nchp + ci) * 4);
  }

  // ---- 4. rows: the next one's loads out, then this one's slice sum into `part`
  const int zadd = a.zeros ? 0 : 8;
  auto row_part = [&](const PacedStage<NIT> &st, int row) {
    float acc = 0.0f;
#pragma unroll
    for (int it = 0; it < NIT; it++) {
      const uint32_t ci = cb + (uint32_t)lane + kWave * it;
      if constexpr (kW16) {
        const int z = (int)paced_byte<F, DW>(st.z[it], ci) + zadd;
        acc = __builtin_fmaf(__uint_as_float(st.s[it]), w4a16_chunk(st.w[it], xv[it], z), acc);
      } else {
        float wl[16], wh[16];
        mxfp4_decode(st.w[it], wl, wh);
        acc = __builtin_fmaf(e8m0_to_f32(paced_byte<F, DW>(st.s[it], ci)), chunk_dot(wl, wh, xv[it]), acc);
      }
    }
    const float t = wave_sum(acc);
    if (lane == 0) part[(row - wr0) * S + sl] = t;
  };
  int r = r0;
  for (; r + 2 < r1; r += 2) {
    paced_load<F, NIT, DW>(a, st1, r + 1, r1, lane, nch, G, cb);
    __builtin_amdgcn_sched_barrier(0);
    row_part(st0, r);
    __builtin_amdgcn_sched_barrier(0);
    paced_load<F, NIT, DW>(a, st0, r + 2, r1, lane, nch, G, cb);
    __builtin_amdgcn_sched_barrier(0);
    row_part(st1, r + 1);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (r + 1 < r1) {
    paced_load<F, NIT, DW>(a, st1, r + 1, r1, lane, nch, G, cb);
    __builtin_amdgcn_sched_barrier(0);
    row_part(st0, r);
    __builtin_amdgcn_sched_barrier(0);
    row_part(st1, r + 1);
  } else if (r < r1) {
    row_part(st0, r);
  }
  // ---- 5. the workgroup's rows: slice sums added in slice order
  __syncthreads();
  for (int i = threadIdx.x; i < wn; i += T) {
    float t = part[i * S];
    for (int s2 = 1; s2 < S; s2++) t += part[i * S + s2];
    a.y[wr0 + i] = t;
  }
}

// LDS of the split kernel: the fp32 activation planes of S whole slices, then the
// workgroup's row sums (rows_max rows x S slices).
inline size_t gemv_split_lds_bytes(int Kp, int rows_max) {
  const int S = ((Kp >> 5) + kSplitChunks - 1) / kSplitChunks;
  return (size_t)S * kSplitChunks * 128 + (size_t)rows_max * S * sizeof(float);
}

// Whether the paced kernel runs this launch: one activation row, no fused prologue or
// epilogue, rows longer than 1024 elements (shorter ones load two rows per wave load
// in gemv_kernel); every format, int4 of either group size.
inline bool gemv_paced_eligible(const GemmArgs &a) {
  return a.M == 1 && gemv_prologue(a) == 0 && !a.bias && !a.res && !a.amax_key && !a.glu && (a.Kp >> 5) > kWave / 2;
}

// Rows held at once (R) from the share of rows each wave gets under the
// persistent grid, for NIT register-held chunks per lane.
// A chosen instantiation: the kernel, its weight rows held per batch (R slots; two
// rows each under HW) and its 16-byte chunks per lane per row.
struct GemvPick {
  GemvFn fn = nullptr;
  int R = 0, nit = 0;
  bool hw = false;
};

template <int F, int MB, int R, int NIT, int PRO, bool HW = false>
static GemvPick gemv_pick() {
  GemvPick p;
  p.fn = gemv_kernel<F, MB, R, NIT, PRO, HW>;
  p.R = R;
  p.nit = NIT;
  p.hw = HW;
  return p;
}

template <int F, int MB, int NIT, int PRO>
static GemvPick pick_gemv_nit(int rpw) {
  // rows held at once: R * NIT chunks of weights must stay in registers next to the
  // activations (larger shares are processed R rows at a time)
  constexpr int RMAX = MB == 1 ? (NIT >= 8 ? 1 : NIT >= 4 ? 2 : 4) : MB == 2 ? (NIT >= 4 ? 1 : 2) : 1;
  if constexpr (RMAX == 1) {
    return gemv_pick<F, MB, 1, NIT, PRO>();
  } else if constexpr (RMAX == 2) {
    return rpw <= 1 ? gemv_pick<F, MB, 1, NIT, PRO>() : gemv_pick<F, MB, 2, NIT, PRO>();
  } else {
    if (rpw <= 1) return gemv_pick<F, MB, 1, NIT, PRO>();
    if (rpw <= 2) return gemv_pick<F, MB, 2, NIT, PRO>();
    if (rpw <= 3) return gemv_pick<F, MB, 3, NIT, PRO>();
    return gemv_pick<F, MB, 4, NIT, PRO>();
  }
}

// Two rows per wave load (HW) for rows of at most 32 chunks: R slots of two rows.
template <int F, int PRO>
static GemvPick pick_gemv_hw(int rpw) {
  const int slots = (rpw + 1) / 2;
  if (slots <= 1) return gemv_pick<F, 1, 1, 1, PRO, true>();
  if (slots <= 2) return gemv_pick<F, 1, 2, 1, PRO, true>();
  if (slots <= 3) return gemv_pick<F, 1, 3, 1, PRO, true>();
  return gemv_pick<F, 1, 4, 1, PRO, true>();
}

// The kernel for rows of nit register-held chunks per lane (nch chunks); no kernel
// (fn null) where the activations exceed the LDS budget.
template <int F, int MB, int PRO>
static GemvPick pick_gemv(int nit, int nch, int rpw) {
  if constexpr (MB == 1 && !fmt_g32(F)) {
    if (nch <= kWave / 2 && rpw >= 2) return pick_gemv_hw<F, PRO>(rpw);
  }
  if constexpr (PRO == 3) {
    return nit <= 1 ? pick_gemv_nit<F, MB, 1, PRO>(rpw) : GemvPick();
  } else {
    if (nit <= 1) return pick_gemv_nit<F, MB, 1, PRO>(rpw);
    if (nit <= 2) return pick_gemv_nit<F, MB, 2, PRO>(rpw);
    if (nit <= 4) return pick_gemv_nit<F, MB, 4, PRO>(rpw);
    // fp32 activations of two or more rows longer than 8192 exceed the LDS budget
    if constexpr ((F == F_W4A16 || F == F_MXFP4 || F == F_W4A16G32) && MB >= 2) return GemvPick();
    else return pick_gemv_nit<F, MB, 8, PRO>(rpw);
  }
}

// The paced kernel: two workgroups per CU where two fit at once, otherwise one.
template <int F>
static hipError_t launch_gemv_paced(const GemmArgs &a, int cus, size_t lds, hipStream_t s, GemvPlan *plan) {
  const int nit = ((a.Kp >> 5) + kWave - 1) / kWave;
  // metadata bytes per row: E8M0 or zero-points one per group (32 or 128 elements)
  const bool dw = ((a.Kp / fmt_group(F)) % 4) == 0;
  if constexpr (F == F_W4A16 || F == F_W4A16G32 || F == F_MXFP4) {
    // rows of more than 4096 elements: split over the waves, where the planes of
    // whole slices stay within the GEMV's LDS budget (rows up to 12288 elements)
    if (nit > 2 && gemv_split_lds_bytes(a.Kp, 0) <= kGemvLdsLimit) {
      const int S = ((a.Kp >> 5) + kSplitChunks - 1) / kSplitChunks;
      // waves per workgroup: the same number for every slice. Three slices: 12 waves
      // (one workgroup per CU) against 8 (slices of 3, 3 and 2 waves, the last
      // slice's waves taking half the rows each): 1 x 4096 x 11008 cold W4A16 8.0 ->
      // 7.5 us, MXFP4 8.0 -> 7.5, 5-15 % at 4096 x 9000 and 11008 x 11008. Two slices:
      // MXFP4 16 waves (one workgroup per CU) against 8 (two): 4096 x 8192 cold 5.7
      // -> 5.2 us; W4A16 stays at 8 (16 measured 0-5 % slower)
      constexpr int kW2 = F == F_MXFP4 ? 16 : kGemvWaves, kW3 = 12;
      const int WV = S == 3 ? kW3 : kW2;
      const GemvFn k = S == 3 ? (dw ? gemv_paced_split_kernel<F, true, kW3, 3> : gemv_paced_split_kernel<F, false, kW3, 3>)
                              : (dw ? gemv_paced_split_kernel<F, true, kW2> : gemv_paced_split_kernel<F, false, kW2>);
      // Workgroups of WV rows each (S row-slices per wave) while they fill the CUs.
      // Fewer rows than that: the fewest row-slices per wave q that the CUs allow,
      // over the fewest workgroups that give it (at most one per CU). 1 x 1024 x
      // 11008 cold W4A16 6.0 -> 4.2 us (86 -> 256 workgroups), MXFP4 5.7 -> 4.4;
      // 1 x 896 x 4864 W4A16 4.2 -> 3.7, MXFP4 4.6 -> 3.8. A workgroup per CU
      // without fewer row-slices per wave only adds activation staging
      // (1 x 1536 x 5000 W4A16 192 -> 256 workgroups: 4.35 -> 4.45 us).
      const int pmin = WV / S;  // waves of the slice with the fewest
      int per_cu = 2, grid = 0;
      size_t slds = 0;
      for (;;) {
        grid = (a.N + WV - 1) / WV;
        if (grid < cus) {
          const int q = (a.N + cus * pmin - 1) / (cus * pmin);
          grid = (a.N + q * pmin - 1) / (q * pmin);
        }
        grid = grid < per_cu * cus ? grid : per_cu * cus;
        slds = gemv_split_lds_bytes(a.Kp, (a.N + grid - 1) / grid);
        if (per_cu == 1 || gemv_wg_per_cu(reinterpret_cast<const void *>(k), slds, WV * kWave) >= 2) break;
        per_cu = 1;
      }
      if (plan) {
        plan->workgroups = grid;
        plan->rows_per_wave = ((a.N + grid - 1) / grid + pmin - 1) / pmin;
        plan->rows_held = 2;
        plan->chunks_per_lane = 2;
        plan->two_rows_per_load = 0;
        plan->act_rows = 1;
        plan->k_slices = S;
        return hipSuccess;
      }
      GemmArgs arg = a;
      arg.split_base = a.N / grid;
      arg.split_rem = a.N % grid;
      void *args[] = {&arg};
      const hipError_t e = hipLaunchKernel(reinterpret_cast<const void *>(k), dim3(grid), dim3(WV * kWave), args,
                                           slds, s);
      return e != hipSuccess ? e : hipGetLastError();
    }
  }
  GemvFn k = nullptr;
  int nk = 0;
  if (nit <= 1) k = dw ? gemv_paced_kernel<F, 1, true> : gemv_paced_kernel<F, 1, false>, nk = 1;
  else if (nit <= 2) k = dw ? gemv_paced_kernel<F, 2, true> : gemv_paced_kernel<F, 2, false>, nk = 2;
  else if (nit <= 4) k = dw ? gemv_paced_kernel<F, 4, true> : gemv_paced_kernel<F, 4, false>, nk = 4;
  else k = dw ? gemv_paced_kernel<F, 8, true> : gemv_paced_kernel<F, 8, false>, nk = 8;
  int per_cu = 2;
  if (gemv_wg_per_cu(reinterpret_cast<const void *>(k), lds) < 2) per_cu = 1;
  int grid = (a.N + kGemvWaves - 1) / kGemvWaves;
  grid = grid < per_cu * cus ? grid : per_cu * cus;
  if (plan) {
    const int waves = grid * kGemvWaves;
    plan->workgroups = grid;
    plan->rows_per_wave = (a.N + waves - 1) / waves;
    plan->rows_held = 2;  // the row being computed and the next one in flight
    plan->chunks_per_lane = nk;
    plan->two_rows_per_load = 0;
    plan->act_rows = 1;
    return hipSuccess;
  }
  GemmArgs arg = a;
  arg.split_base = a.N / grid;
  arg.split_rem = a.N % grid;
  void *args[] = {&arg};
  const hipError_t e = hipLaunchKernel(reinterpret_cast<const void *>(k), dim3(grid), dim3(kGemvThreads), args, lds, s);
  return e != hipSuccess ? e : hipGetLastError();
}

// Persistent grid of at most two workgroups per CU, fewer when there are few rows.
// Two only when two fit on a CU at once (at most 128 VGPRs per lane, and the LDS of
// both): otherwise the second waits for the first to finish, and one workgroup per
// CU with twice the rows is faster (long rows: 9-16 % at 1 x 4096 x 11008 cold).
// W4A8 quantizes the activation row in every workgroup, so below two rows per wave
// it takes one workgroup per CU as well (3-9 % at N = 3072 .. 6144), and so does a
// W4A8 GEMV with a prologue whose workgroups would get under 32 KB of weights.
template <int F, int MB, int PRO>
static hipError_t launch_gemv_mb(const GemmArgs &a, int num_cus, size_t lds, hipStream_t s, GemvPlan *plan) {
  constexpr bool kQuant = (F == F_W4A8 || F == F_W4A8G32);
  const int nit = ((a.Kp >> 5) + kWave - 1) / kWave;
  const int cus = num_cus > 0 ? num_cus : 256;
  // W4A8 with a fused prologue (RMSNorm before the quantizer) and a small share of
  // weights per workgroup: the prologue, not the weight stream, sets the time, and
  // it runs faster with the CU to itself (gate/up 9728 x 896: 5.1 -> 4.5 us)
  const double wg_bytes = (double)a.N * (a.Kp / 2) / (2.0 * cus);
  int per_cu = (kQuant && (a.N < 2 * 2 * cus * kGemvWaves || (PRO != 0 && wg_bytes < 32768.0))) ? 1 : 2;
  if constexpr (MB == 1 && PRO == 0) {
    if (gemv_paced_eligible(a)) return launch_gemv_paced<F>(a, cus, lds, s, plan);
  }
  for (;;) {
    int grid = (a.N + kGemvWaves - 1) / kGemvWaves;
    grid = grid < per_cu * cus ? grid : per_cu * cus;
    const int waves = grid * kGemvWaves;
    const int rpw = a.glu ? 2 * ((a.N / 2 + waves - 1) / waves) : (a.N + waves - 1) / waves;
    const GemvPick pk = pick_gemv<F, MB, PRO>(nit, a.Kp >> 5, rpw);
    const GemvFn k = pk.fn;
    if (!k) return hipErrorInvalidValue;
    if (per_cu == 2 && grid > cus && gemv_wg_per_cu(reinterpret_cast<const void *>(k), lds) < 2) {
      per_cu = 1;
      continue;
    }
    if (plan) {
      plan->workgroups = grid;
      plan->rows_per_wave = rpw;
      plan->rows_held = pk.hw ? 2 * pk.R : pk.R;
      plan->chunks_per_lane = pk.nit;
      plan->two_rows_per_load = pk.hw ? 1 : 0;
      plan->act_rows = MB;
      return hipSuccess;
    }
    GemmArgs arg = a;
    void *args[] = {&arg};
    const hipError_t e = hipLaunchKernel(reinterpret_cast<const void *>(k), dim3(grid), dim3(kGemvThreads), args,
                                         lds, s);
    return e != hipSuccess ? e : hipGetLastError();
  }
}

template <int F>
static hipError_t launch_gemv_f(const GemmArgs &a, int num_cus, size_t lds, hipStream_t s, GemvPlan *plan) {
  const int pro = gemv_prologue(a);
  if (pro != 0) {
    if (a.M != 1 || (a.norm_w && a.swiglu)) return hipErrorInvalidValue;
    // the prologues act on fp32 rows, and the group-32 formats have none
    if constexpr (F == F_W4A8Q || fmt_g32(F)) return hipErrorInvalidValue;
    else if (pro == 1) return launch_gemv_mb<F, 1, 1>(a, num_cus, lds, s, plan);
    else if (pro == 2) return launch_gemv_mb<F, 1, 2>(a, num_cus, lds, s, plan);
    else if (a.Kp > kWave * 32) return hipErrorInvalidValue;  // one chunk per lane
    else return launch_gemv_mb<F, 1, 3>(a, num_cus, lds, s, plan);
  }
  switch (a.M) {
    case 1: return launch_gemv_mb<F, 1, 0>(a, num_cus, lds, s, plan);
    case 2: return launch_gemv_mb<F, 2, 0>(a, num_cus, lds, s, plan);
    case 3: return launch_gemv_mb<F, 3, 0>(a, num_cus, lds, s, plan);
    case 4: return launch_gemv_mb<F, 4, 0>(a, num_cus, lds, s, plan);
  }
  return hipErrorInvalidValue;
}

}  // namespace lbk
