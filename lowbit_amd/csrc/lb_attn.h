// One decode token's attention for one query head, as device functions of the
// one-token attention kernel (lb_model.hip): src/lowbit/model.py:353-378 for a
// single query at absolute position p against the KV-cache keys 0 .. S-1,
// S = min(p + 1, cap), where (when p < cap) key p is the new one, held in
// registers and never read back from the cache.
//
// Exponentials of the softmax and of the merges are the hardware's (__expf: their
// arguments are <= 0, and a few ulp of exp(x) stay far inside the attention bound).
//
// Memory layout of the work: D / 4 lanes share a key (or value) row, each lane
// holding one float4 of it, so a wave load covers RPL = 256 / D consecutive rows
// (1 KiB contiguous). A wave takes KB = 16 RPL keys per round (16 key loads and 16
// value loads per lane, all in flight together, within the 63 loads a wave can
// have outstanding): the score of each key is a sum over its row's lanes, and
// the lanes that hold a value row already hold that key's probability. Every
// wave keeps its own online softmax (running max, sum and p * v) over rounds
// of NW * KB keys; the waves are merged once at the end, in LDS. The first
// round's rows are requested before the position is known (rows below cap).
#pragma once

#include <math.h>

#include "lb_device.h"

namespace lbk {

template <int D, int UU = 16>
struct AttnCfg {
  static constexpr int kLPR = D / 4;          // lanes per key row
  static constexpr int kRPL = kWave / kLPR;   // key rows per wave load
  static constexpr int kU = UU;               // key (and value) loads per lane and round
  static constexpr int kKB = kU * kRPL;       // keys per wave and round
};

// Key slices (of KB keys) that hold keys below S, at least one, at most NS.
__host__ __device__ __forceinline__ int attn_active_slices(int S, int KB, int NS) {
  const int n = (S + KB - 1) / KB;
  return n < 1 ? 1 : (n < NS ? n : NS);
}

// Registers holding one round of a wave's key and value rows.
template <int D, int UU = 16>
struct AttnRound {
  float4 k[AttnCfg<D, UU>::kU];
  float4 v[AttnCfg<D, UU>::kU];
};

// LDS of the final merge for NT threads.
template <int D, int NT>
struct AttnShared {
  float part[NT / kWave][D];  // per-wave p * v sums
  float mw[NT / kWave];       // per-wave running maxima
  float lw[NT / kWave];       // per-wave softmax sums
};

// Sum over each group of LPR consecutive lanes (8, 16 or 32); every lane of the
// group gets it.
template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
  v += dpp_f<kDppQuad1032>(v, 0.0f);
  v += dpp_f<kDppQuad2301>(v, 0.0f);
  v += dpp_f<kDppRowHalfMirror>(v, 0.0f);  // 8-lane sums
  if constexpr (LPR >= 16) v += dpp_f<kDppRowMirror>(v, 0.0f);
  if constexpr (LPR >= 32) v += __shfl_xor(v, 16);
  return v;
}

// Sum over the lanes l, l + LPR, l + 2 LPR, ... (the same element of every row a
// wave load covers); every lane gets its column's sum.
template <int LPR>
__device__ __forceinline__ float column_sum(float v) {
#pragma unroll
  for (int off = LPR; off < kWave; off <<= 1) v += __shfl_xor(v, off);
  return v;
}

// Key and value rows of one round of this wave, starting at key k0; rows clamped
// below cap, so every address is inside the cache (rows past the keys in use are
// masked out of the softmax). kb / vb: the KV head's cache rows [cap][D].
template <int D, int UU = 16>
__device__ __forceinline__ void attn_load_round(AttnRound<D, UU> &rd, const float *__restrict__ kb,
                                                const float *__restrict__ vb, int k0, int cap) {
  constexpr int LPR = AttnCfg<D, UU>::kLPR, RPL = AttnCfg<D, UU>::kRPL, U = AttnCfg<D, UU>::kU;
  const int lane = threadIdx.x & (kWave - 1), r = lane / LPR, e4 = lane % LPR;
#pragma unroll
  for (int u = 0; u < U; u++) {
    int row = k0 + RPL * u + r;
    row = row < cap ? row : cap - 1;
    rd.k[u] = reinterpret_cast<const float4 *>(kb + (size_t)row * D)[e4];
  }
#pragma unroll
  for (int u = 0; u < U; u++) {
    int row = k0 + RPL * u + r;
    row = row < cap ? row : cap - 1;
    rd.v[u] = reinterpret_cast<const float4 *>(vb + (size_t)row * D)[e4];
  }
}

// The first round of this wave (keys KB * wave ...), issued by the caller before
// anything else.
template <int D, int NT>
__device__ __forceinline__ void attn_prefetch(AttnRound<D> &rd, const float *__restrict__ kb,
                                              const float *__restrict__ vb, int cap) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  attn_load_round<D>(rd, kb, vb, AttnCfg<D>::kKB * wave, cap);
}

// Attention of the rotated query over keys 0 .. S-1: keys other than Sc from the
// cache rows kb / vb, key Sc (when newk) the new one. Each lane passes its float4
// (elements 4 (lane % (D/4)) ..) of the rotated query q4, the new key kn4 and its
// value vn4. `first` holds the wave's first round (attn_prefetch). Writes
// out[0 .. D). Every thread of the workgroup calls it (one barrier, at the merge).
template <int D, int NT>
__device__ __forceinline__ void attn_run(const AttnRound<D> &first, float4 q4, float4 kn4, float4 vn4,
                                         const float *__restrict__ kb, const float *__restrict__ vb, int S,
                                         int Sc, bool newk, int cap, AttnShared<D, NT> &sh,
                                         float *__restrict__ out) {
  constexpr int LPR = AttnCfg<D>::kLPR, RPL = AttnCfg<D>::kRPL, U = AttnCfg<D>::kU, KB = AttnCfg<D>::kKB;
  constexpr int NW = NT / kWave;
  static_assert(NT % kWave == 0, "whole waves");
  const int tid = threadIdx.x, lane = tid & (kWave - 1), r = lane / LPR;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const float scale = 1.0f / sqrtf((float)D);
  float m = -INFINITY, l = 0.0f;
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  AttnRound<D> rd = first;
  for (int c0 = 0; c0 < S; c0 += NW * KB) {
    const int k0 = c0 + KB * wave;
    if (c0 > 0) attn_load_round<D>(rd, kb, vb, k0, cap);
    if (k0 >= S) continue;  // wave-uniform: no key of this round for this wave
    // ---- scores of the round's keys (each in all lanes of its row)
    float sc[U];
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int row = k0 + RPL * u + r;
      const float4 kk = (newk && row == Sc) ? kn4 : rd.k[u];
      float d = q4.x * kk.x;
      d = __builtin_fmaf(q4.y, kk.y, d);
      d = __builtin_fmaf(q4.z, kk.z, d);
      d = __builtin_fmaf(q4.w, kk.w, d);
      d = group_sum<LPR>(d) * scale;
      sc[u] = row < S ? d : -INFINITY;
      mx = fmaxf(mx, sc[u]);
    }
    // ---- running maximum (the round has a key below S: row k0), rescale, p * v
    const float mnew = fmaxf(m, wave_max(mx));
    const float alpha = __expf(m - mnew);  // 0 on the wave's first round
    m = mnew;
    l *= alpha;
    acc.x *= alpha;
    acc.y *= alpha;
    acc.z *= alpha;
    acc.w *= alpha;
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int row = k0 + RPL * u + r;
      const float pr = __expf(sc[u] - m);  // 0 for masked keys
      // masked rows (past the keys in use) may hold anything, NaN included: 0 * NaN
      // would poison the sum, so their values are replaced, not just weighted by 0
      const float4 vv = row < S ? ((newk && row == Sc) ? vn4 : rd.v[u]) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      l += pr;
      acc.x = __builtin_fmaf(pr, vv.x, acc.x);
      acc.y = __builtin_fmaf(pr, vv.y, acc.y);
      acc.z = __builtin_fmaf(pr, vv.z, acc.z);
      acc.w = __builtin_fmaf(pr, vv.w, acc.w);
    }
  }
  // ---- the wave's sums over its rows, then the waves merged in LDS
  acc.x = column_sum<LPR>(acc.x);
  acc.y = column_sum<LPR>(acc.y);
  acc.z = column_sum<LPR>(acc.z);
  acc.w = column_sum<LPR>(acc.w);
  l = column_sum<LPR>(l);  // each row's sum is held by all its lanes
  if (lane < LPR) *reinterpret_cast<float4 *>(&sh.part[wave][4 * lane]) = acc;
  if (lane == 0) {
    sh.mw[wave] = m;
    sh.lw[wave] = l;
  }
  __syncthreads();
  float M = sh.mw[0];
#pragma unroll
  for (int w = 1; w < NW; w++) M = fmaxf(M, sh.mw[w]);
  for (int e = tid; e < D; e += NT) {
    float num = 0.0f, den = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; w++) {
      const float f = __expf(sh.mw[w] - M);  // 0 for a wave that saw no key
      num = __builtin_fmaf(sh.part[w][e], f, num);
      den = __builtin_fmaf(sh.lw[w], f, den);
    }
    out[e] = num / den;
  }
}

// Partials of up to 8 key slices of one head, for the float4 at elements 4 e4 ..:
// p * v, max and sum of each (attn_fetch8), combined by attn_combine8.
struct AttnPart8 {
  float4 a[8];
  float m[8], l[8];
};

// Slices s0 .. s0 + 7 of the head's partials ph (PS floats each: p * v [D], max,
// sum; ph and PS keep every partial 16-byte aligned); slots past slice n - 1 read
// slice n - 1 again. All loads issued together.
__device__ __forceinline__ void attn_fetch8(AttnPart8 &q, const float *ph, int PS, int D, int s0, int n, int e4) {
#pragma unroll
  for (int b = 0; b < 8; b++) {
    const int s = s0 + b < n ? s0 + b : n - 1;
    q.a[b] = *reinterpret_cast<const float4 *>(ph + (size_t)s * PS + 4 * e4);
    const float2 ml = *reinterpret_cast<const float2 *>(ph + (size_t)s * PS + D);  // max and sum: one load
    q.m[b] = ml.x;
    q.l[b] = ml.y;
  }
}

// Adds slices s0 .. min(s0 + 8, n) - 1 of q, weighted by exp(m - M), to num / den
// in slice order.
__device__ __forceinline__ void attn_combine8(const AttnPart8 &q, int s0, int n, float M, float4 &num, float &den) {
#pragma unroll
  for (int b = 0; b < 8; b++) {
    if (s0 + b >= n) break;
    const float f = __expf(q.m[b] - M);
    num.x = __builtin_fmaf(q.a[b].x, f, num.x);
    num.y = __builtin_fmaf(q.a[b].y, f, num.y);
    num.z = __builtin_fmaf(q.a[b].z, f, num.z);
    num.w = __builtin_fmaf(q.a[b].w, f, num.w);
    den = __builtin_fmaf(q.l[b], f, den);
  }
}

// The merged float4 of at most 8 slices already fetched: sum_s acc_s f_s /
// sum_s l_s f_s, f_s = exp(m_s - M), M = max_s m_s.
__device__ __forceinline__ float4 attn_merge8(const AttnPart8 &q, int n) {
  float M = -INFINITY;
#pragma unroll
  for (int b = 0; b < 8; b++) M = fmaxf(M, q.m[b]);  // repeats of the last slice change nothing
  float4 num = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  float den = 0.0f;
  attn_combine8(q, 0, n, M, num, den);
  const float rd = 1.0f / den;
  return make_float4(num.x * rd, num.y * rd, num.z * rd, num.w * rd);
}

// Elements 4 e4 .. 4 e4 + 3 of one head's attention output from the partials of its
// n key slices (the same arithmetic as attn_merge8 for n <= 8, where it is one
// round trip; more slices take two passes of 8 at a time).
__device__ __forceinline__ float4 attn_merge4(const float *ph, int PS, int D, int n, int e4) {
  AttnPart8 q;
  attn_fetch8(q, ph, PS, D, 0, n, e4);
  if (n <= 8) return attn_merge8(q, n);
  float M = -INFINITY;
  for (int s0 = 0; s0 < n; s0 += 8) {
    if (s0) attn_fetch8(q, ph, PS, D, s0, n, e4);
#pragma unroll
    for (int b = 0; b < 8; b++) M = fmaxf(M, q.m[b]);
  }
  float4 num = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  float den = 0.0f;
  for (int s0 = 0; s0 < n; s0 += 8) {
    attn_fetch8(q, ph, PS, D, s0, n, e4);
    attn_combine8(q, s0, n, M, num, den);
  }
  const float rd = 1.0f / den;
  return make_float4(num.x * rd, num.y * rd, num.z * rd, num.w * rd);
}

// Rotate the pair (x1, x2) of element i of a head at the table row pc
// ("rotate_half", src/lowbit/model.py:201-210): each product rounded, then the
// sum, as numpy's float32 evaluates it (no fused multiply-add, so every kernel
// that inlines this gives the same bits).
__device__ __forceinline__ void rope_pair(float x1, float x2, float c, float s, float &y1, float &y2) {
#pragma clang fp contract(off)
  y1 = x1 * c - x2 * s;
  y2 = x2 * c + x1 * s;
}

// The rotated value of one element of a head: `own` is the element, `partner`
// the one it is paired with (i + D/2 for i < D/2, i - D/2 otherwise; `hi` for the
// second half), c / s the angle of the pair.
__device__ __forceinline__ float rope_elem(bool hi, float own, float partner, float c, float s) {
  float y1, y2;
  rope_pair(hi ? partner : own, hi ? own : partner, c, s, y1, y2);
  return hi ? y2 : y1;
}

// Elements 4 e4 .. 4 e4 + 3 of the head row x [D] rotated at table row pc (cos/sin
// tables [.., D/2]); x, the tables and their rows 16-byte aligned.
template <int D>
__device__ __forceinline__ float4 rope4(const float *x, const float *__restrict__ cosT,
                                        const float *__restrict__ sinT, int pc, int e4) {
  constexpr int half = D / 2;
  static_assert(half % 4 == 0, "a float4 never straddles the two halves");
  const int e = 4 * e4;
  const bool hi = e >= half;
  const int i = hi ? e - half : e;
  const float4 a = *reinterpret_cast<const float4 *>(x + e);
  const float4 b = *reinterpret_cast<const float4 *>(x + (hi ? i : e + half));
  const float4 c = *reinterpret_cast<const float4 *>(cosT + (size_t)pc * half + i);
  const float4 s = *reinterpret_cast<const float4 *>(sinT + (size_t)pc * half + i);
  return make_float4(rope_elem(hi, a.x, b.x, c.x, s.x), rope_elem(hi, a.y, b.y, c.y, s.y),
                     rope_elem(hi, a.z, b.z, c.z, s.z), rope_elem(hi, a.w, b.w, c.w, s.w));
}

}  // namespace lbk
