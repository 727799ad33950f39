// One decode token's attention for one query head, as device functions shared by
// the one-token attention kernel (lb_model.hip) and the fused q/k/v GEMV +
// attention kernel (lb_gemv.h): src/lowbit/model.py:353-378 for a single query at
// absolute position p against the KV-cache keys 0 .. S-1, S = min(p + 1, cap),
// where (when p < cap) key p is the new one, held in LDS and never read back from
// the cache.
//
// NT threads (NT / 64 waves) per workgroup; keys are scored NT per chunk (one per
// thread) with an online softmax across chunks; wave w accumulates p * v over keys
// c0 + 64 w .. c0 + 64 w + 63 of a chunk, lane l owning output elements l, l + 64,
// ...; the waves' partial sums are added in LDS at the end. The kernel memory
// chain is short when the first chunk's key and value rows are prefetched into
// registers before anything else (attn_prefetch, D <= 64).
#pragma once

#include <math.h>

#include "lb_device.h"

namespace lbk {

template <int D>
struct AttnCfg {
  static constexpr int kDPL = (D + kWave - 1) / kWave;  // output elements per lane
  static constexpr bool kPre = D <= 64;                  // first chunk prefetched into registers
  static constexpr int kVB = 16;                         // values in flight per lane past the first chunk
};

// Registers holding the first chunk's key row (one per thread) and value rows (64
// per wave) of the workgroup's KV head.
template <int D>
struct AttnPre {
  float4 k[AttnCfg<D>::kPre ? D / 4 : 1];
  float v[AttnCfg<D>::kPre ? kWave * AttnCfg<D>::kDPL : 1];
};

// LDS of attn_run for NT threads.
template <int D, int NT>
struct AttnShared {
  float pb[NT];                   // probabilities of the chunk's keys
  float red[NT / kWave];          // per-wave chunk maxima
  float part[NT / kWave][D];      // per-wave partial outputs
  float lsw[NT / kWave];          // per-wave softmax sums
};

// Issue the prefetch (rows clamped below cap, so every address is in the cache;
// rows past the keys in use are loaded but never used). kb / vb: the KV head's
// cache rows [cap][D].
template <int D, int NT>
__device__ __forceinline__ void attn_prefetch(AttnPre<D> &pre, const float *__restrict__ kb,
                                              const float *__restrict__ vb, int cap) {
  if constexpr (AttnCfg<D>::kPre) {
    constexpr int DPL = AttnCfg<D>::kDPL;
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    const int l = (D >= kWave || lane < D) ? lane : 0;
    const int t = tid < cap ? tid : cap - 1;
    const float4 *kr = reinterpret_cast<const float4 *>(kb + (size_t)t * D);
#pragma unroll
    for (int e = 0; e < D / 4; e++) pre.k[e] = kr[e];
#pragma unroll
    for (int u = 0; u < kWave; u++) {
      const int row = wave * kWave + u < cap ? wave * kWave + u : cap - 1;
#pragma unroll
      for (int q = 0; q < DPL; q++) pre.v[u * DPL + q] = vb[(size_t)row * D + l + kWave * q];
    }
  }
}

// Attention of the rotated query qs[D] (LDS) over keys 0 .. S-1: keys below Sc from
// the cache rows kb / vb, key Sc (when newk) from kn / vn (LDS). Writes out[0 .. D).
// Every thread of the workgroup calls it (it has barriers); the LDS in qs, kn, vn
// must be visible to all threads on entry.
template <int D, int NT>
__device__ __forceinline__ void attn_run(const AttnPre<D> &pre, const float *qs, const float *kn, const float *vn,
                                         const float *__restrict__ kb, const float *__restrict__ vb, int S,
                                         int Sc, bool newk, AttnShared<D, NT> &sh, float *__restrict__ out) {
  constexpr int DPL = AttnCfg<D>::kDPL, NK4 = D / 4, NW = NT / kWave, VB = AttnCfg<D>::kVB;
  constexpr bool kPre = AttnCfg<D>::kPre;
  static_assert(NT % kWave == 0 && NT >= kWave, "whole waves");
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const bool own = D >= kWave || lane < D;  // D = 32: lanes 32..63 hold no output
  const int l = own ? lane : 0;
  const float scale = 1.0f / sqrtf((float)D);
  float acc[DPL], lsum = 0.0f, mrun = -INFINITY;
#pragma unroll
  for (int q = 0; q < DPL; q++) acc[q] = 0.0f;

  for (int c0 = 0; c0 < S; c0 += NT) {
    const bool pre_chunk = kPre && c0 == 0;
    // ---- score of key c0 + tid
    const int s = c0 + tid;
    float d = 0.0f;
    if (s < S) {
      float4 kv[NK4];
      if (s >= Sc) {
#pragma unroll
        for (int e = 0; e < NK4; e++) kv[e] = reinterpret_cast<const float4 *>(kn)[e];
      } else if (pre_chunk) {
#pragma unroll
        for (int e = 0; e < NK4; e++) kv[e] = pre.k[kPre ? e : 0];
      } else {
        const float4 *kr = reinterpret_cast<const float4 *>(kb + (size_t)s * D);
#pragma unroll
        for (int e = 0; e < NK4; e++) kv[e] = kr[e];
      }
#pragma unroll
      for (int e = 0; e < NK4; e++) {
        const float4 qv = reinterpret_cast<const float4 *>(qs)[e];
        d = __builtin_fmaf(qv.x, kv[e].x, d);
        d = __builtin_fmaf(qv.y, kv[e].y, d);
        d = __builtin_fmaf(qv.z, kv[e].z, d);
        d = __builtin_fmaf(qv.w, kv[e].w, d);
      }
    }
    d = s < S ? d * scale : -INFINITY;
    const float mw = wave_max(d);
    if (lane == 0) sh.red[wave] = mw;
    __syncthreads();
    // ---- running maximum, probabilities of this chunk, rescaled accumulators
    float cm = sh.red[0];
#pragma unroll
    for (int w = 1; w < NW; w++) cm = fmaxf(cm, sh.red[w]);
    const float mnew = fmaxf(mrun, cm);
    const float alpha = expf(mrun - mnew);  // 0 on the first chunk
    mrun = mnew;
    lsum *= alpha;
#pragma unroll
    for (int q = 0; q < DPL; q++) acc[q] *= alpha;
    sh.pb[tid] = s < S ? expf(d - mnew) : 0.0f;
    __syncthreads();
    // ---- wave w: p * v over keys c0 + 64 w .. c0 + 64 w + 63; the new key's
    //      value from LDS
    const int sb = c0 + wave * kWave;
    const int se = sb + kWave < S ? sb + kWave : S;
    const int sce = se < Sc ? se : Sc;
    if (pre_chunk) {
#pragma unroll
      for (int u = 0; u < kWave; u++) {
        if (sb + u < sce) {
          const float pr = sh.pb[sb + u - c0];
          lsum += pr;
#pragma unroll
          for (int q = 0; q < DPL; q++) acc[q] = __builtin_fmaf(pr, pre.v[kPre ? u * DPL + q : 0], acc[q]);
        }
      }
    } else {
      for (int k0 = sb; k0 < sce; k0 += VB) {
        float v[VB][DPL];
#pragma unroll
        for (int u = 0; u < VB; u++) {
          const int k = k0 + u < sce ? k0 + u : sce - 1;  // in-range row; its weight is dropped below
#pragma unroll
          for (int q = 0; q < DPL; q++) v[u][q] = vb[(size_t)k * D + l + kWave * q];
        }
#pragma unroll
        for (int u = 0; u < VB; u++) {
          if (k0 + u < sce) {
            const float pr = sh.pb[k0 + u - c0];
            lsum += pr;
#pragma unroll
            for (int q = 0; q < DPL; q++) acc[q] = __builtin_fmaf(pr, v[u][q], acc[q]);
          }
        }
      }
    }
    if (newk && Sc >= sb && Sc < se) {
      const float pr = sh.pb[Sc - c0];
      lsum += pr;
#pragma unroll
      for (int q = 0; q < DPL; q++) acc[q] = __builtin_fmaf(pr, vn[l + kWave * q], acc[q]);
    }
    __syncthreads();  // pb is rewritten by the next chunk
  }

  // ---- add the waves' partial sums
  if (own) {
#pragma unroll
    for (int q = 0; q < DPL; q++) sh.part[wave][l + kWave * q] = acc[q];
  }
  if (lane == 0) sh.lsw[wave] = lsum;
  __syncthreads();
  for (int e = tid; e < D; e += NT) {
    float num = 0.0f, den = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; w++) {
      num += sh.part[w][e];
      den += sh.lsw[w];
    }
    out[e] = num / den;
  }
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

}  // namespace lbk
