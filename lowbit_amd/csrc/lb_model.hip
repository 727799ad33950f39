// Decoder-layer kernels around the fused GEMMs, for a device-resident decoder
// (Qwen2 / Llama architecture of the reference's numpy model, src/lowbit/model.py):
// embedding gather, RMSNorm, q/k/v bias + rotary embedding + KV-cache write,
// grouped-query causal attention, SwiGLU, residual add and greedy argmax.
//
// Activations are fp32 row-major [T, width]. The decode position and the current
// token live in device memory (`pos`, `tok`), so one decode step is a fixed
// sequence of launches that a HIP graph can replay: the kernels read the position
// from `pos`, and the argmax writes the next token and advances `pos`.
#include <math.h>

#include <type_traits>

#include "lb_device.h"
#include "lb_attn.h"
#include "lb_internal.h"

namespace lbk {

constexpr int kMT = 256;  // threads of the row kernels

// Sum over a workgroup of kMT threads; every thread gets the result.
__device__ __forceinline__ float block_sum(float v, float *red) {
  v = wave_sum(v);
  const int w = threadIdx.x / kWave;
  __syncthreads();  // red may still be read from a previous call
  if ((threadIdx.x & (kWave - 1)) == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < kMT / kWave; i++) r += red[i];
  return r;
}

// x[t] = table[tok[t]] (token ids clamped into the table).
__global__ __launch_bounds__(kMT) void embed_kernel(const float *__restrict__ table, int vocab, int hidden,
                                                     const int32_t *__restrict__ tok, float *__restrict__ x) {
  const int t = blockIdx.x;
  int id = tok[t];
  id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);
  const float *src = table + (size_t)id * hidden;
  for (int i = threadIdx.x; i < hidden; i += kMT) x[(size_t)t * hidden + i] = src[i];
}

// y = x * (1 / sqrt(mean(x^2) + eps)) * w, one workgroup per row (the reference's
// rms_norm, src/lowbit/model.py:190-192, in float32).
__global__ __launch_bounds__(kMT) void rmsnorm_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                       int hidden, float eps, float *__restrict__ y) {
  __shared__ float red[kMT / kWave];
  const float *xr = x + (size_t)blockIdx.x * hidden;
  float ss = 0.0f;
  for (int i = threadIdx.x; i < hidden; i += kMT) ss = __builtin_fmaf(xr[i], xr[i], ss);
  const float var = block_sum(ss, red) / (float)hidden;
  const float r = 1.0f / sqrtf(var + eps);
  for (int i = threadIdx.x; i < hidden; i += kMT) y[(size_t)blockIdx.x * hidden + i] = xr[i] * r * w[i];
}

// qkv [T, (H + 2 KV) D]: adds the bias, rotates q and k at absolute position
// pos + t (the "rotate_half" convention: element i pairs with i + D/2,
// src/lowbit/model.py:201-210) with the float32 tables cos/sin [max_pos, D/2], leaves
// q in place and writes k and v into the caches [KV, cap, D]. One workgroup per
// (token, head), D/2 threads.
__global__ void qkv_rope_kernel(float *__restrict__ qkv, const float *__restrict__ bias, int H, int KV, int D,
                                const float *__restrict__ cosT, const float *__restrict__ sinT,
                                const int32_t *__restrict__ pos, int max_pos, float *__restrict__ kc,
                                float *__restrict__ vc, int cap) {
  const int t = blockIdx.x, hd = blockIdx.y, i = threadIdx.x, half = D / 2;
  const int p = *pos + t;
  if (p < 0) return;  // no position before the start of the cache
  const int width = (H + 2 * KV) * D;
  float *row = qkv + (size_t)t * width + (size_t)hd * D;
  const float *b = bias ? bias + (size_t)hd * D : nullptr;
  float x1 = row[i], x2 = row[i + half];
  if (b) {
    x1 += b[i];
    x2 += b[i + half];
  }
  if (hd < H + KV) {  // q or k: rotate
    const int pp = p < max_pos ? p : max_pos - 1;  // positions past the tables reuse the last angle
    const float c = cosT[(size_t)pp * half + i], s = sinT[(size_t)pp * half + i];
    float y1, y2;
    rope_pair(x1, x2, c, s, y1, y2);
    x1 = y1;
    x2 = y2;
  }
  if (hd < H) {
    row[i] = x1;
    row[i + half] = x2;
  } else if (p < cap) {
    const int kvh = hd < H + KV ? hd - H : hd - H - KV;
    float *dst = (hd < H + KV ? kc : vc) + ((size_t)kvh * cap + p) * D;
    dst[i] = x1;
    dst[i + half] = x2;
  }
}

// Causal grouped-query attention: query t (absolute position pos + t) of head h
// against keys 0 .. pos + t of KV head h / (H / KV), softmax(q k^T / sqrt(D)) v
// (src/lowbit/model.py:353-378). One workgroup of one wave per (token, head):
// scores one key per lane into LDS, wave max and sum, then lane l owns output
// elements l, l + 64, ... below D. q rows have stride qstride floats; out is [T, H D].
template <int D>
__global__ __launch_bounds__(kWave) void attention_kernel(const float *__restrict__ q, int qstride,
                                                          const float *__restrict__ kc,
                                                          const float *__restrict__ vc, int H, int KV,
                                                          const int32_t *__restrict__ pos, int cap,
                                                          float *__restrict__ out) {
  extern __shared__ float sc[];  // [cap] scores, then [D] query
  constexpr int DPL = (D + kWave - 1) / kWave;
  const int t = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
  const int kvh = h / (H / KV);
  int S = *pos + t + 1;
  S = S < cap ? S : cap;
  float *qs = sc + cap;
  const float *qr = q + (size_t)t * qstride + (size_t)h * D;
  for (int e = lane; e < D; e += kWave) qs[e] = qr[e];
  __syncthreads();
  const float scale = 1.0f / sqrtf((float)D);
  const float *kb = kc + (size_t)kvh * cap * D;
  float mx = -INFINITY;
  for (int s = lane; s < S; s += kWave) {
    const float4 *kr = reinterpret_cast<const float4 *>(kb + (size_t)s * D);
    float d = 0.0f;
#pragma unroll 4
    for (int e = 0; e < D / 4; e++) {
      const float4 kv = kr[e];
      d = __builtin_fmaf(qs[4 * e], kv.x, d);
      d = __builtin_fmaf(qs[4 * e + 1], kv.y, d);
      d = __builtin_fmaf(qs[4 * e + 2], kv.z, d);
      d = __builtin_fmaf(qs[4 * e + 3], kv.w, d);
    }
    d *= scale;
    sc[s] = d;
    mx = fmaxf(mx, d);
  }
  mx = wave_max(mx);
  float sum = 0.0f;
  for (int s = lane; s < S; s += kWave) {
    const float e = expf(sc[s] - mx);
    sc[s] = e;
    sum += e;
  }
  sum = wave_sum(sum);
  __syncthreads();
  const float inv = 1.0f / sum;
  const float *vb = vc + (size_t)kvh * cap * D;
  const bool own = D >= kWave || lane < D;  // D = 32: lanes 32..63 hold no output
  const int l = own ? lane : 0;
  float acc[DPL];
#pragma unroll
  for (int j = 0; j < DPL; j++) acc[j] = 0.0f;
  for (int s = 0; s < S; s++) {
    const float ps = sc[s];
#pragma unroll
    for (int j = 0; j < DPL; j++) acc[j] = __builtin_fmaf(ps, vb[(size_t)s * D + l + kWave * j], acc[j]);
  }
  if (own) {
#pragma unroll
    for (int j = 0; j < DPL; j++) out[(size_t)t * H * D + (size_t)h * D + l + kWave * j] = acc[j] * inv;
  }
}

// One-token attention (the decode step) with the rotary embedding and the KV-cache
// write folded in: the q / k / v row of the token (bias already added by the GEMM
// epilogue) sits in qkv [(H + 2 KV) D] at absolute position p = *pos. One workgroup
// per query head h (grid KV x H/KV; KV head g = h / (H/KV)). The step is a chain
// of memory round trips, so the kernel is laid out to need as few as possible:
//   0. before anything else (and before *pos arrives) each wave requests its first
//      round of key and value rows (coalesced float4 rows, lb_attn.h; rows below
//      cap);
//   1. every lane rotates its float4 of the query head and of the key
//      ("rotate_half", src/lowbit/model.py:201-210) in registers, with no LDS and
//      no barrier; the group's first workgroup writes the rotated key and the
//      value to the caches at p (when p < cap);
//   2. every wave runs an online softmax over its keys of each round
//      (src/lowbit/model.py:353-378), with no barrier;
//   3. the waves' (max, sum, p * v) are merged in LDS and divided by the sum.
// Keys 0 .. S-1 with S = min(p + 1, cap) take part; when p < cap key p is the new
// one (from registers, never read back from the cache), otherwise all S come from the
// cache, as lbd_qkv_rope + lbd_attention behave. Output out [H D].
constexpr int kAttThreads = 256;

template <int D>
__global__ __launch_bounds__(kAttThreads) void attention_decode_kernel(
    const float *__restrict__ qkv, int H, int KV, const float *__restrict__ cosT, const float *__restrict__ sinT,
    const int32_t *__restrict__ pos, int max_pos, float *__restrict__ kc, float *__restrict__ vc, int cap,
    float *__restrict__ out) {
  __shared__ AttnShared<D, kAttThreads> sh;
  const int g = blockIdx.x, j = blockIdx.y, HG = gridDim.y, h = g * HG + j;
  const int tid = threadIdx.x, e4 = tid % (D / 4);
  const float *kb = kc + (size_t)g * cap * D;
  const float *vb = vc + (size_t)g * cap * D;

  // ---- 0. the first round of keys and values, requested before anything else
  AttnRound<D> pre;
  attn_prefetch<D, kAttThreads>(pre, kb, vb, cap);

  const int p = *pos;
  const int pc = p < 0 ? 0 : (p < max_pos ? p : max_pos - 1);  // positions past the tables reuse the last angle
  const bool newk = p >= 0 && p < cap;
  const int S = p < 0 ? 0 : (p + 1 < cap ? p + 1 : cap);
  const int Sc = newk ? S - 1 : S;  // keys read from the cache; key Sc is the new one when newk

  // ---- 1. every lane rotates its float4 of the query head and of the key; the
  //         group's first workgroup writes the key and the value to the caches
  const float4 q4 = rope4<D>(qkv + (size_t)h * D, cosT, sinT, pc, e4);
  const float4 kn4 = rope4<D>(qkv + (size_t)(H + g) * D, cosT, sinT, pc, e4);
  const float4 vn4 = *reinterpret_cast<const float4 *>(qkv + (size_t)(H + KV + g) * D + 4 * e4);
  if (newk && j == 0 && tid < D / 4) {
    *reinterpret_cast<float4 *>(kc + ((size_t)g * cap + p) * D + 4 * e4) = kn4;
    *reinterpret_cast<float4 *>(vc + ((size_t)g * cap + p) * D + 4 * e4) = vn4;
  }

  // ---- 2, 3. per-wave online softmax over rounds of keys; the waves merged
  attn_run<D, kAttThreads>(pre, q4, kn4, vn4, kb, vb, S, Sc, newk, cap, sh, out + (size_t)h * D);
}

// Key slices: the same one-token attention with each query head's keys cut into
// slices of one wave round (KB keys, lb_attn.h; 8 loads per lane and round, i.e.
// 2048 / D keys, where 8 such slices hold the cache, else 16) on one-wave workgroups, grid
// KV x H/KV x NS, so that a head's keys stream through NS compute units instead of
// one. Workgroup (g, j, sl) takes the rounds sl, sl + NS, ... below S and stores
// its (p * v, max, sum) partial; attention_merge_kernel (long caches) or the fused
// GEMVs' attention-merge prologue (the decoder's o projection) combines them after
// the kernel boundary (no fence, no counter: an in-kernel merge through an
// agent-scope fence and an atomic cost more than the split saved). The slices
// holding keys below 256 request their first round before *pos arrives; slices
// past the keys in use store an empty partial (max -inf, sum 0) without loading
// anything, so that a merge may take all slices. Rotation and the cache write are
// those of attention_decode_kernel.
constexpr int kAttnPrefetchKeys = 256;

template <int D, int UU>
__global__ __launch_bounds__(kWave) void attention_slice_kernel(
    const float *__restrict__ qkv, int H, int KV, const float *__restrict__ cosT, const float *__restrict__ sinT,
    const int32_t *__restrict__ pos, int max_pos, float *__restrict__ kc, float *__restrict__ vc, int cap,
    float *__restrict__ part) {
  using Cfg = AttnCfg<D, UU>;
  constexpr int LPR = Cfg::kLPR, RPL = Cfg::kRPL, U = Cfg::kU, KB = Cfg::kKB, PS = D + 4;
  const int g = blockIdx.x, j = blockIdx.y, HG = gridDim.y, h = g * HG + j;
  const int sl = blockIdx.z, NS = gridDim.z;
  const int lane = threadIdx.x, r = lane / LPR, e4 = lane % LPR;
  const float *kb = kc + (size_t)g * cap * D;
  const float *vb = vc + (size_t)g * cap * D;
  // the slices holding keys below 256 request their first round before *pos arrives
  AttnRound<D, UU> rd;
  const bool early = KB * sl < kAttnPrefetchKeys;
  if (early) attn_load_round<D, UU>(rd, kb, vb, KB * sl, cap);
  const int p = *pos;
  const int pc = p < 0 ? 0 : (p < max_pos ? p : max_pos - 1);
  const bool newk = p >= 0 && p < cap;
  const int S = p < 0 ? 0 : (p + 1 < cap ? p + 1 : cap);
  const int Sc = newk ? S - 1 : S;
  float *pp = part + ((size_t)h * NS + sl) * PS;
  if (sl >= attn_active_slices(S, KB, NS)) {
    // no key: an empty partial (weight exp(-inf) = 0 in any merge over all slices)
    if (r == 0) *reinterpret_cast<float4 *>(pp + 4 * e4) = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (lane == 0) {
      pp[D] = -INFINITY;
      pp[D + 1] = 0.0f;
    }
    return;
  }
  if (!early) attn_load_round<D, UU>(rd, kb, vb, KB * sl, cap);
  const float4 q4 = rope4<D>(qkv + (size_t)h * D, cosT, sinT, pc, e4);
  const float4 kn4 = rope4<D>(qkv + (size_t)(H + g) * D, cosT, sinT, pc, e4);
  const float4 vn4 = *reinterpret_cast<const float4 *>(qkv + (size_t)(H + KV + g) * D + 4 * e4);
  if (newk && j == 0 && sl == 0 && r == 0) {
    *reinterpret_cast<float4 *>(kc + ((size_t)g * cap + p) * D + 4 * e4) = kn4;
    *reinterpret_cast<float4 *>(vc + ((size_t)g * cap + p) * D + 4 * e4) = vn4;
  }
  const float scale = 1.0f / sqrtf((float)D);
  float m = -INFINITY, l = 0.0f;
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (int c = sl; KB * c < S; c += NS) {
    const int k0 = KB * c;
    if (c != sl) attn_load_round<D, UU>(rd, kb, vb, k0, cap);
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
    const float mnew = fmaxf(m, wave_max(mx));  // the round has a key below S: row k0
    const float alpha = __expf(m - mnew);       // 0 on the first round
    m = mnew;
    l *= alpha;
    acc.x *= alpha;
    acc.y *= alpha;
    acc.z *= alpha;
    acc.w *= alpha;
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int row = k0 + RPL * u + r;
      const float pr = __expf(sc[u] - m);
      // masked rows may hold anything, NaN included: their values are replaced
      const float4 vv = row < S ? ((newk && row == Sc) ? vn4 : rd.v[u]) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      l += pr;
      acc.x = __builtin_fmaf(pr, vv.x, acc.x);
      acc.y = __builtin_fmaf(pr, vv.y, acc.y);
      acc.z = __builtin_fmaf(pr, vv.z, acc.z);
      acc.w = __builtin_fmaf(pr, vv.w, acc.w);
    }
  }
  acc.x = column_sum<LPR>(acc.x);
  acc.y = column_sum<LPR>(acc.y);
  acc.z = column_sum<LPR>(acc.z);
  acc.w = column_sum<LPR>(acc.w);
  l = column_sum<LPR>(l);
  if (r == 0) *reinterpret_cast<float4 *>(pp + 4 * e4) = acc;
  if (lane == 0) {
    pp[D] = m;
    pp[D + 1] = l;
  }
}

// out[h] = the slices' partials of head h combined. Up to 8 active slices:
// attn_merge8, the arithmetic of the attention-merge prologue of the fused GEMVs
// (so that both give the same bits). More (long caches): every load is issued
// before the first wait (lane s holds slice s's max and sum, and the partial
// vectors are read for all kAttnMaxSplit slots, slots past the active slices
// re-reading the last one with weight 0), so the merge costs one round trip, not
// one per group of slices. One wave per head.
template <int D>
__global__ __launch_bounds__(kWave) void attention_merge_kernel(const int32_t *__restrict__ pos, int cap, int NS,
                                                                int KB, const float *__restrict__ part,
                                                                float *__restrict__ out) {
  static_assert(kAttnMaxSplit <= kWave, "one lane per slice");
  constexpr int LPR = D / 4, PS = D + 4;
  const int h = blockIdx.x, lane = threadIdx.x, e4 = lane % LPR;
  const int p = *pos;
  const int S = p < 0 ? 0 : (p + 1 < cap ? p + 1 : cap);
  const int nact = attn_active_slices(S, KB, NS);
  const float *ph = part + (size_t)h * NS * PS;
  float4 *o4 = reinterpret_cast<float4 *>(out + (size_t)h * D) + e4;
  if (nact <= 8) {
    if (lane >= LPR) return;
    AttnPart8 q;
    attn_fetch8(q, ph, PS, D, 0, nact, e4);
    *o4 = attn_merge8(q, nact);
    return;
  }
  float4 a[kAttnMaxSplit];
#pragma unroll
  for (int s = 0; s < kAttnMaxSplit; s++)
    a[s] = *reinterpret_cast<const float4 *>(ph + (size_t)(s < nact ? s : nact - 1) * PS + 4 * e4);
  const int sl = lane < nact ? lane : nact - 1;
  const float2 ml = *reinterpret_cast<const float2 *>(ph + (size_t)sl * PS + D);
  const float M = wave_max(lane < nact ? ml.x : -INFINITY);
  const float f = lane < nact ? __expf(ml.x - M) : 0.0f;
  const float den = wave_sum(ml.y * f);
  float4 num = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
  for (int s = 0; s < kAttnMaxSplit; s++) {
    const float fs = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f), s));  // 0 past the active slices
    num.x = __builtin_fmaf(a[s].x, fs, num.x);
    num.y = __builtin_fmaf(a[s].y, fs, num.y);
    num.z = __builtin_fmaf(a[s].z, fs, num.z);
    num.w = __builtin_fmaf(a[s].w, fs, num.w);
  }
  const float rd = 1.0f / den;
  if (lane < LPR) *o4 = make_float4(num.x * rd, num.y * rd, num.z * rd, num.w * rd);
}

// tok[0] = the index of the largest of the kArgmaxSlots keys that lbd_gemv_*_fused
// max-combined (the one argmax_kernel would pick from the logits); advances *pos
// and records hist[*pos] like argmax_kernel, and clears every slot for the next
// step. One workgroup of 256 threads, four slots each.
constexpr int kFinT = 256;
__global__ __launch_bounds__(kFinT) void argmax_finalize_kernel(unsigned long long *__restrict__ key,
                                                                int32_t *__restrict__ tok, int32_t *__restrict__ pos,
                                                                int inc, int32_t *__restrict__ hist, int hist_len) {
  static_assert(kArgmaxSlots == 4 * kFinT, "four slots per thread");
  __shared__ unsigned long long wbest[kFinT / kWave];
  unsigned long long b = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const unsigned long long k = key[threadIdx.x + i * kFinT];
    b = k > b ? k : b;
  }
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const unsigned long long o = __shfl_xor(b, off);
    b = o > b ? o : b;
  }
  if ((threadIdx.x & (kWave - 1)) == 0) wbest[threadIdx.x / kWave] = b;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; i++) key[threadIdx.x + i * kFinT] = 0;
  if (threadIdx.x == 0) {
    for (int w = 1; w < kFinT / kWave; w++) b = wbest[w] > b ? wbest[w] : b;
    const int ix = argmax_key_index(b);
    tok[0] = ix;
    if (pos) {
      const int p = *pos + inc;
      if (hist && p >= 0 && p < hist_len) hist[p] = ix;
      *pos = p;
    }
  }
}

// out[t, i] = silu(gu[t, i]) * gu[t, I + i], silu(g) = g / (1 + exp(-g))
// (src/lowbit/model.py:213, 416-417).
__global__ __launch_bounds__(kMT) void swiglu_kernel(const float *__restrict__ gu, int T, int I,
                                                      float *__restrict__ out) {
  const size_t n = (size_t)T * I;
  for (size_t e = (size_t)blockIdx.x * kMT + threadIdx.x; e < n; e += (size_t)gridDim.x * kMT) {
    const size_t t = e / I, i = e % I;
    const float g = gu[t * 2 * I + i], u = gu[t * 2 * I + I + i];
    out[e] = g / (1.0f + expf(-g)) * u;
  }
}

// out[t, i] = silu(gu[t, 2i]) * gu[t, 2i + 1]: gate and up interleaved by output.
__global__ __launch_bounds__(kMT) void swiglu_pairs_kernel(const float *__restrict__ gu, size_t n,
                                                            float *__restrict__ out) {
  for (size_t e = (size_t)blockIdx.x * kMT + threadIdx.x; e < n; e += (size_t)gridDim.x * kMT) {
    const float2 p = reinterpret_cast<const float2 *>(gu)[e];
    out[e] = p.x / (1.0f + expf(-p.x)) * p.y;
  }
}

__global__ __launch_bounds__(kMT) void add_kernel(float *__restrict__ x, const float *__restrict__ y, size_t n) {
  for (size_t e = (size_t)blockIdx.x * kMT + threadIdx.x; e < n; e += (size_t)gridDim.x * kMT) x[e] += y[e];
}

// numpy's argmax order: NaN above every number, then larger values, then the
// smaller index among equals.
__device__ __forceinline__ bool argmax_before(float a, int ia, float b, int ib) {
  const bool na = a != a, nb = b != b;
  if (na || nb) return na && (!nb || ia < ib);
  return a > b || (a == b && ia < ib);
}

// Index of the largest value as numpy's argmax picks it (the first NaN if there is
// one, else the first maximum). One workgroup of 1024 threads. Writes the index to
// tok[0] and, with pos != null, stores it into hist[*pos + inc] (when inside
// hist_len) and advances *pos by inc.
constexpr int kAT = 1024;
__global__ __launch_bounds__(kAT) void argmax_kernel(const float *__restrict__ v, int n, int32_t *__restrict__ tok,
                                                      int32_t *__restrict__ pos, int inc, int32_t *__restrict__ hist,
                                                      int hist_len) {
  __shared__ float bv[kAT / kWave];
  __shared__ int bi[kAT / kWave];
  float best = -INFINITY;
  int bidx = 0x7FFFFFFF;
  for (int i = threadIdx.x; i < n; i += kAT) {
    const float x = v[i];
    if (argmax_before(x, i, best, bidx)) best = x, bidx = i;
  }
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const float ov = __shfl_xor(best, off);
    const int oi = __shfl_xor(bidx, off);
    if (argmax_before(ov, oi, best, bidx)) best = ov, bidx = oi;
  }
  const int w = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) bv[w] = best, bi[w] = bidx;
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = bv[0];
    int ix = bi[0];
    for (int k = 1; k < kAT / kWave; k++)
      if (argmax_before(bv[k], bi[k], b, ix)) b = bv[k], ix = bi[k];
    if (ix == 0x7FFFFFFF) ix = 0;  // n == 0
    tok[0] = ix;
    if (pos) {
      const int p = *pos + inc;
      if (hist && p >= 0 && p < hist_len) hist[p] = ix;
      *pos = p;
    }
  }
}

// ---------------------------------------------------------------- launchers

static unsigned grid_for(size_t n) {
  size_t b = (n + kMT - 1) / kMT;
  if (b > 16384) b = 16384;
  return (unsigned)(b ? b : 1);
}

hipError_t launch_embed(const float *table, int vocab, int hidden, const int32_t *tok, int T, float *x, hipStream_t s) {
  hipLaunchKernelGGL(embed_kernel, dim3(T), dim3(kMT), 0, s, table, vocab, hidden, tok, x);
  return hipGetLastError();
}

hipError_t launch_rmsnorm(const float *x, const float *w, int T, int hidden, float eps, float *y, hipStream_t s) {
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(T), dim3(kMT), 0, s, x, w, hidden, eps, y);
  return hipGetLastError();
}

hipError_t launch_qkv_rope(float *qkv, const float *bias, int T, int H, int KV, int D, const float *cosT,
                           const float *sinT, const int32_t *pos, int max_pos, float *kc, float *vc, int cap,
                           hipStream_t s) {
  hipLaunchKernelGGL(qkv_rope_kernel, dim3(T, H + 2 * KV), dim3(D / 2), 0, s, qkv, bias, H, KV, D, cosT, sinT, pos,
                     max_pos, kc, vc, cap);
  return hipGetLastError();
}

hipError_t launch_attention(const float *q, int qstride, const float *kc, const float *vc, int T, int H, int KV, int D,
                            const int32_t *pos, int cap, float *out, hipStream_t s) {
  const size_t lds = ((size_t)cap + D) * sizeof(float);
  if (D == 32)
    hipLaunchKernelGGL(attention_kernel<32>, dim3(T, H), dim3(kWave), lds, s, q, qstride, kc, vc, H, KV, pos, cap, out);
  else if (D == 64)
    hipLaunchKernelGGL(attention_kernel<64>, dim3(T, H), dim3(kWave), lds, s, q, qstride, kc, vc, H, KV, pos, cap, out);
  else if (D == 128)
    hipLaunchKernelGGL(attention_kernel<128>, dim3(T, H), dim3(kWave), lds, s, q, qstride, kc, vc, H, KV, pos, cap,
                       out);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_swiglu(const float *gu, int T, int I, float *out, hipStream_t s) {
  hipLaunchKernelGGL(swiglu_kernel, dim3(grid_for((size_t)T * I)), dim3(kMT), 0, s, gu, T, I, out);
  return hipGetLastError();
}

hipError_t launch_swiglu_pairs(const float *gu, int T, int I, float *out, hipStream_t s) {
  const size_t n = (size_t)T * I;
  hipLaunchKernelGGL(swiglu_pairs_kernel, dim3(grid_for(n)), dim3(kMT), 0, s, gu, n, out);
  return hipGetLastError();
}

hipError_t launch_add(float *x, const float *y, size_t n, hipStream_t s) {
  hipLaunchKernelGGL(add_kernel, dim3(grid_for(n)), dim3(kMT), 0, s, x, y, n);
  return hipGetLastError();
}

hipError_t launch_argmax(const float *v, int n, int32_t *tok, int32_t *pos, int inc, int32_t *hist, int hist_len,
                         hipStream_t s) {
  hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(kAT), 0, s, v, n, tok, pos, inc, hist, hist_len);
  return hipGetLastError();
}

hipError_t launch_attention_slices(const float *qkv, int H, int KV, int D, const float *cosT, const float *sinT,
                                   const int32_t *pos, int max_pos, float *kc, float *vc, int cap, float *part,
                                   hipStream_t s) {
  if (KV <= 0 || H % KV || H / KV > kAttnMaxGroup || cap <= 0) return hipErrorInvalidValue;
  const dim3 grid(KV, H / KV, attn_slices(D, cap));
  const bool half = attn_slice_keys(D, cap) * D == 32 * kWave;  // 8 loads per lane and round
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(kWave), 0, s, qkv, H, KV, cosT, sinT, pos, max_pos, kc, vc, cap, part);
    return hipGetLastError();
  };
  if (D == 32) return half ? go(attention_slice_kernel<32, 8>) : go(attention_slice_kernel<32, 16>);
  if (D == 64) return half ? go(attention_slice_kernel<64, 8>) : go(attention_slice_kernel<64, 16>);
  if (D == 128) return half ? go(attention_slice_kernel<128, 8>) : go(attention_slice_kernel<128, 16>);
  return hipErrorInvalidValue;
}

hipError_t launch_attention_merge(const float *part, int H, int D, const int32_t *pos, int cap, float *out,
                                  hipStream_t s) {
  if (H <= 0 || cap <= 0) return hipErrorInvalidValue;
  const int ns = attn_slices(D, cap), kb = attn_slice_keys(D, cap);
  if (D == 32)
    hipLaunchKernelGGL(attention_merge_kernel<32>, dim3(H), dim3(kWave), 0, s, pos, cap, ns, kb, part, out);
  else if (D == 64)
    hipLaunchKernelGGL(attention_merge_kernel<64>, dim3(H), dim3(kWave), 0, s, pos, cap, ns, kb, part, out);
  else if (D == 128)
    hipLaunchKernelGGL(attention_merge_kernel<128>, dim3(H), dim3(kWave), 0, s, pos, cap, ns, kb, part, out);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_attention_decode(const float *qkv, int H, int KV, int D, const float *cosT, const float *sinT,
                                   const int32_t *pos, int max_pos, float *kc, float *vc, int cap, float *out,
                                   float *work, hipStream_t s) {
  if (KV <= 0 || H % KV || H / KV > kAttnMaxGroup || cap <= 0) return hipErrorInvalidValue;
  if (work && cap >= kAttnSliceMinCap) {
    const hipError_t e = launch_attention_slices(qkv, H, KV, D, cosT, sinT, pos, max_pos, kc, vc, cap, work, s);
    if (e != hipSuccess) return e;
    return launch_attention_merge(work, H, D, pos, cap, out, s);
  }
  const dim3 grid(KV, H / KV);
  if (D == 32)
    hipLaunchKernelGGL(attention_decode_kernel<32>, grid, dim3(kAttThreads), 0, s, qkv, H, KV, cosT, sinT, pos,
                       max_pos, kc, vc, cap, out);
  else if (D == 64)
    hipLaunchKernelGGL(attention_decode_kernel<64>, grid, dim3(kAttThreads), 0, s, qkv, H, KV, cosT, sinT, pos,
                       max_pos, kc, vc, cap, out);
  else if (D == 128)
    hipLaunchKernelGGL(attention_decode_kernel<128>, grid, dim3(kAttThreads), 0, s, qkv, H, KV, cosT, sinT, pos,
                       max_pos, kc, vc, cap, out);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_argmax_finalize(unsigned long long *key, int32_t *tok, int32_t *pos, int inc, int32_t *hist,
                                  int hist_len, hipStream_t s) {
  hipLaunchKernelGGL(argmax_finalize_kernel, dim3(1), dim3(kFinT), 0, s, key, tok, pos, inc, hist, hist_len);
  return hipGetLastError();
}

}  // namespace lbk
