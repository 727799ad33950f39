// gfx950 (MI355X, CDNA4) kernels for the fused dequantize + GEMM
//     Y[M,N] = X[M,Kp] . W[N,Kp]^T
// over the packed int4-g128 and MXFP4 layouts (src/lowbit/csrc/lowbit.h:9-19).
//
// Regimes
//   gemv_kernel       M <= 4: HBM-bound. Each lane streams 16 contiguous bytes of
//                     a weight row (32 codes) per step, decodes them in registers
//                     and reduces across the wave. No LDS for weights, no MFMA.
//                     X (or, for W4A8, the int8 codes the fused quantizer
//                     produces) sits in LDS in "plane" order so that the 32
//                     activations a lane needs for its 16 bytes are eight (or
//                     two) conflict-free 16-byte LDS reads.
//   w4a8_mfma_kernel  W4A8 for larger M: v_mfma_i32_16x16x64_i8 on the int8
//                     activations and the (q - z) bytes, giving the exact int32
//                     group accumulator per 16x16 tile, then an fp32 rescale.
//   f32_mfma_kernel   W4A16 / MXFP4 for larger M: v_mfma_f32_16x16x4_f32 with the
//                     exactly decoded weights, so products and sums keep fp32
//                     semantics.
//   quant_rows_kernel the per-token int8 quantizer (one workgroup per row).
//
// MFMA operand mapping. For a 16x16xK MFMA, lane l supplies row (l % 16) of A and
// column (l % 16) of B for the k-slots owned by lane group q = l / 16; the
// hardware pairs slot t of A with slot t of B within the same lane group. Which
// actual k a slot holds is therefore free, as long as A and B agree. Each lane
// loads 16 contiguous bytes of a weight row (the natural packed order) and puts
// the matching activations in the same slots, so weights go from HBM to the
// matrix cores without an LDS transpose.
#include <algorithm>
#include <map>
#include <mutex>
#include <utility>

#include <type_traits>

#include "lb_device.h"
#include "lb_gemv.h"
#include "lb_internal.h"

namespace lbk {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

// ============================================================ per-token quantizer
//
// Tiled int8 activation layout (internal to the W4A8 MFMA path): rows in blocks of
// 16, each (row block, group, half) a 1 KiB tile holding the 16-byte MFMA operand
// of every lane in lane order, so that the GEMM reads each operand with one fully
// contiguous 1 KiB wave load. Element e of row m (group g = e / 128, r = e % 128,
// half h = r / 64, lane group q = (r % 64) / 16) sits at byte
//   (((m / 16 * G + g) * 2 + h) * 64 + 16 q + m % 16) * 16 + r % 16.
// The group sums of the tiled path are stored [m / 16][g][m % 16].
__device__ __forceinline__ uint32_t w4a8_tiled_offset(int m, int e, int G) {
  const int g = e >> 7, r = e & 127;
  return (uint32_t)((((((m >> 4) * G + g) * 2 + (r >> 6)) * 64 + ((r >> 4) & 3) * 16 + (m & 15)) * 16) + (r & 15));
}
//
// One workgroup per activation row. With NR > 0 the row (at most NR * 1024
// elements) is loaded into registers by NR unconditional 16-byte loads per thread
// (offsets past the row read 0), so all loads are in flight together; NR == 0
// streams longer rows twice. The absmax is reduced across the workgroup and each
// thread quantizes its 4-element slots with the exact fast path; group sums land
// in asum.
template <int NR, bool TILED>
__global__ __launch_bounds__(kThreads) void quant_rows_kernel(
    const float *__restrict__ x, int M, int Kp, int8_t *__restrict__ xq, float *__restrict__ xs,
    int32_t *__restrict__ asum) {
  __shared__ float red[kWaves];
  const int m = blockIdx.x;
  const int G = Kp / kGroup;
  if (TILED && m >= M) {
    // padding rows of the last 16-row block: zero codes and sums
    for (int e = threadIdx.x * 4; e < Kp; e += kThreads * 4)
      *reinterpret_cast<uint32_t *>(xq + w4a8_tiled_offset(m, e, G)) = 0u;
    for (int g = threadIdx.x; g < G; g += kThreads) asum[((m >> 4) * G + g) * 16 + (m & 15)] = 0;
    return;
  }
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const Rsrc rx = make_rsrc(x + (size_t)m * Kp, (uint32_t)Kp * 4);
  float4 v[NR > 0 ? NR : 1];
  float amax = 0.0f;
  if constexpr (NR > 0) {
#pragma unroll
    for (int i = 0; i < NR; i++) v[i] = ld_f4(rx, (threadIdx.x + i * kThreads) * 16);
#pragma unroll
    for (int i = 0; i < NR; i++) {
      amax = fmaxf(fmaxf(amax, fabsf(v[i].x)), fabsf(v[i].y));
      amax = fmaxf(fmaxf(amax, fabsf(v[i].z)), fabsf(v[i].w));
    }
  } else {
    for (int e = threadIdx.x * 4; e < Kp; e += kThreads * 4) {
      const float4 t = ld_f4(rx, e * 4);
      amax = fmaxf(fmaxf(amax, fabsf(t.x)), fabsf(t.y));
      amax = fmaxf(fmaxf(amax, fabsf(t.z)), fabsf(t.w));
    }
  }
  amax = wave_max(amax);
  if (lane == 0) red[wave] = amax;
  __syncthreads();
  float rmax = red[0];
#pragma unroll
  for (int w = 1; w < kWaves; w++) rmax = fmaxf(rmax, red[w]);
  const float sc = row_scale(rmax);
  const float inv = 1.0f / sc;
  if (threadIdx.x == 0) xs[m] = sc;
  // thread t handles 4 elements per slot; a group of 128 is one 32-lane half-wave
  // (Kp % 128 == 0, so half-waves enter and leave a slot together)
  auto emit = [&](float4 t, int e) {
    const uint32_t qv = quant4_fast(t, sc, inv);
    const int gs = half_wave_sum(sum_i8x4(qv));
    if constexpr (TILED) {
      *reinterpret_cast<uint32_t *>(xq + w4a8_tiled_offset(m, e, G)) = qv;
      if ((threadIdx.x & 31) == 31) asum[((m >> 4) * G + (e >> 7)) * 16 + (m & 15)] = gs;
    } else {
      reinterpret_cast<uint32_t *>(xq + (size_t)m * Kp)[e >> 2] = qv;
      if ((threadIdx.x & 31) == 31) asum[(size_t)m * G + (e >> 7)] = gs;
    }
  };
  if constexpr (NR > 0) {
#pragma unroll
    for (int i = 0; i < NR; i++) {
      const int e = threadIdx.x * 4 + i * kThreads * 4;
      if (e < Kp) emit(v[i], e);
    }
  } else {
    for (int e = threadIdx.x * 4; e < Kp; e += kThreads * 4) emit(ld_f4(rx, e * 4), e);
  }
}

// ============================================================ small-M GEMV (VALU)
//
// The kernels live in lb_gemv.h (shared with the group-32 instantiations).

// Activation planes, then (int8 formats) group sums and row scales.
size_t gemv_lds_bytes(int fmt, int M, int Kp) {
  const size_t nchp = gemv_nchp(Kp);
  if (fmt == F_W4A16 || fmt == F_MXFP4 || fmt == F_W4A16G32) return (size_t)M * nchp * 32 * sizeof(float);
  const size_t groups = fmt_g32(fmt) ? nchp : nchp / 4;  // padded group sums per row
  return (size_t)M * nchp * 32 + (size_t)M * groups * sizeof(int32_t) + 16;
}

bool gemv_eligible(int fmt, int M, int Kp) {
  return M >= 1 && M <= kGemvMaxM && Kp <= kGemvMaxNit * kWave * 32 &&
         gemv_lds_bytes(fmt, M, Kp) <= kGemvLdsLimit;
}

int gemv_wg_per_cu(const void *kern, size_t lds, int threads) {
  static std::mutex mu;
  static std::map<std::pair<const void *, size_t>, int> known;
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_pair(kern, lds);
  const auto it = known.find(key);
  if (it != known.end()) return it->second;
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, threads, lds) != hipSuccess || n < 1) n = 1;
  known[key] = n;
  return n;
}

hipError_t launch_gemv(int fmt, const GemmArgs &a, int num_cus, hipStream_t s, GemvPlan *plan) {
  if (!gemv_eligible(fmt, a.M, a.Kp)) return hipErrorInvalidValue;
  const size_t lds = gemv_lds_bytes(fmt, a.M, a.Kp);
  switch (fmt) {
    case F_W4A16: return launch_gemv_f<F_W4A16>(a, num_cus, lds, s, plan);
    case F_MXFP4: return launch_gemv_f<F_MXFP4>(a, num_cus, lds, s, plan);
    case F_W4A8: return launch_gemv_f<F_W4A8>(a, num_cus, lds, s, plan);
    case F_W4A8Q: return launch_gemv_f<F_W4A8Q>(a, num_cus, lds, s, plan);
    case F_W4A16G32:
    case F_W4A8G32: return launch_gemv_g32(fmt, a, num_cus, lds, s, plan);
  }
  return hipErrorInvalidValue;
}

template <bool TILED>
static void launch_quant_t(const float *x, int M, int Kp, int8_t *xq, float *xs, int32_t *asum, hipStream_t s) {
  const int n4 = (Kp + kThreads * 4 - 1) / (kThreads * 4);  // 16-byte slots per thread
  const dim3 grid(TILED ? (M + 15) / 16 * 16 : M), block(kThreads);
  if (n4 <= 1)
    hipLaunchKernelGGL((quant_rows_kernel<1, TILED>), grid, block, 0, s, x, M, Kp, xq, xs, asum);
  else if (n4 <= 2)
    hipLaunchKernelGGL((quant_rows_kernel<2, TILED>), grid, block, 0, s, x, M, Kp, xq, xs, asum);
  else if (n4 <= 4)
    hipLaunchKernelGGL((quant_rows_kernel<4, TILED>), grid, block, 0, s, x, M, Kp, xq, xs, asum);
  else if (n4 <= 8)
    hipLaunchKernelGGL((quant_rows_kernel<8, TILED>), grid, block, 0, s, x, M, Kp, xq, xs, asum);
  else if (n4 <= 16)
    hipLaunchKernelGGL((quant_rows_kernel<16, TILED>), grid, block, 0, s, x, M, Kp, xq, xs, asum);
  else
    hipLaunchKernelGGL((quant_rows_kernel<0, TILED>), grid, block, 0, s, x, M, Kp, xq, xs, asum);
}

hipError_t launch_quant(const float *x, int M, int Kp, int8_t *xq, float *xs, int32_t *asum, bool tiled,
                        hipStream_t s) {
  if (tiled)
    launch_quant_t<true>(x, M, Kp, xq, xs, asum, s);
  else
    launch_quant_t<false>(x, M, Kp, xq, xs, asum, s);
  return hipGetLastError();
}

// ============================================================ W4A8, int8 MFMA
//
// Persistent workgroups of kW8Waves waves. A workgroup owns a contiguous range of
// 16-row weight subtiles and a block of 16*TM activation rows; its waves split
// the K groups (wave w: kW8GW consecutive groups of each phase of
// kW8Waves * kW8GW groups). Per phase each wave holds its activation slice in
// registers (2 * TM * kW8GW 16-byte operands), so the activations are read
// once per workgroup while the weights stream past:
//   for each subtile (weights prefetched one subtile ahead):
//     two v_mfma_i32_16x16x64_i8 per (row block, group) on the raw codes,
//     acc - z * asum  = the exact int32 group accumulator,
//     fp32 rescale by the group scale,
//   then the waves' partial tiles are summed in LDS in a fixed order (wave 0..7,
//   phase 0..) and scaled by the per-token scale: no atomics, so results do
//   not depend on scheduling.
// With more than one phase (K > kW8Waves * kW8GW * 128) the per-subtile sums of
// earlier phases wait in LDS; subtiles are then processed in passes of at most
// kW8Pass so that this buffer stays bounded.
//
// Operand slots: lane (q = l/16, c = l%16) feeds activation row 16i + c and
// weight row n0 + c with bytes 64g + 16q .. +16 of the group's 64 bytes, i.e.
// elements 128g + 16q + [0, 16) (low nibbles, first MFMA) and 128g + 64 + 16q +
// [0, 16) (high nibbles, second MFMA).

constexpr int kW8Waves = 8;
constexpr int kW8Threads = kW8Waves * kWave;
constexpr int kW8GW = 4;                        // groups per wave per phase
constexpr int kW8Phase = kW8Waves * kW8GW;      // groups per phase
constexpr int kW8Pass = 8;                      // subtiles per pass (multi-phase only)

// Weight bytes, scales and zero-points of one wave's groups for one weight row.
// VEC (G % 4 == 0): the wave's four groups are 4-aligned, so their scales are one
// 16-byte load and their zero-points one dword. Otherwise each group loads its
// scale and the aligned dword holding its zero-point byte (the zero-point
// descriptor is rounded up to whole dwords: the word holding the last byte lies in
// the same page as that byte).
struct W8Stage {
  uint4 w[kW8GW];
  float s[kW8GW];
  uint32_t zw[kW8GW];
};

template <bool VEC>
__device__ __forceinline__ void w8_load(W8Stage &st, Rsrc rw, Rsrc rs, Rsrc rz, int n, int N, int gb, int gcnt,
                                        int G, uint32_t rowbytes, int q) {
#pragma unroll
  for (int t = 0; t < kW8GW; t++) {
    const bool ok = n < N && t < gcnt;
    const uint32_t g = (uint32_t)(gb + t);
    st.w[t] = ld_b128(rw, ok ? (uint32_t)n * rowbytes + g * 64u + (uint32_t)q * 16u : 0xFFFFFFF0u);
  }
  const uint32_t gi0 = (uint32_t)n * (uint32_t)G + (uint32_t)gb;
  if constexpr (VEC) {
    const bool ok = n < N && gcnt > 0;
    const float4 sv = ld_f4(rs, ok ? gi0 * 4u : 0xFFFFFFF0u);
    st.s[0] = sv.x;
    st.s[1] = sv.y;
    st.s[2] = sv.z;
    st.s[3] = sv.w;
    st.zw[0] = ld_u32(rz, ok ? gi0 : 0xFFFFFFF0u);
  } else {
#pragma unroll
    for (int t = 0; t < kW8GW; t++) {
      const bool ok = n < N && t < gcnt;
      st.s[t] = ld_f32(rs, ok ? (gi0 + t) * 4u : 0xFFFFFFF0u);
      st.zw[t] = ld_u32(rz, ok ? ((gi0 + t) & ~3u) : 0xFFFFFFF0u);
    }
  }
}

template <bool VEC>
__device__ __forceinline__ int w8_zero(const W8Stage &st, int t, int n, int G, int gb) {
  if constexpr (VEC) return (int)((st.zw[0] >> (8 * t)) & 0xFFu);
  const uint32_t gi = (uint32_t)n * (uint32_t)G + (uint32_t)(gb + t);
  return (int)((st.zw[t] >> (8u * (gi & 3u))) & 0xFFu);
}

template <int TM, bool VEC, bool EXPORT>
__device__ __forceinline__ void w8_compute(const W8Stage &st, const v4i (&xlo)[kW8GW][TM],
                                           const v4i (&xhi)[kW8GW][TM], const int32_t *as_lds, int gl0,
                                           int gcnt, int zadd, v4f (&facc)[TM], int q, int c, int m0,
                                           int M, int n, int N, int G, int gb, int32_t *__restrict__ out) {
  const v4i zero4 = {0, 0, 0, 0};
#pragma unroll
  for (int t = 0; t < kW8GW; t++) {
    if (t >= gcnt) break;  // wave-uniform
    const v4i blo = {(int)lo_nibbles(st.w[t].x), (int)lo_nibbles(st.w[t].y), (int)lo_nibbles(st.w[t].z),
                     (int)lo_nibbles(st.w[t].w)};
    const v4i bhi = {(int)hi_nibbles(st.w[t].x), (int)hi_nibbles(st.w[t].y), (int)hi_nibbles(st.w[t].z),
                     (int)hi_nibbles(st.w[t].w)};
    const int z = w8_zero<VEC>(st, t, n, G, gb) + zadd;
#pragma unroll
    for (int i = 0; i < TM; i++) {
      v4i acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(xlo[t][i], blo, zero4, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(xhi[t][i], bhi, acc, 0, 0, 0);
      const v4i as = *reinterpret_cast<const v4i *>(as_lds + (gl0 + t) * (16 * TM) + 16 * i + 4 * q);
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int gacc = acc[r] - __mul24(z, as[r]);  // exact: |z * asum| < 2^18
        if constexpr (EXPORT) {
          const int m = m0 + 16 * i + 4 * q + r;
          if (m < M && n < N) out[((size_t)m * N + n) * G + gb + t] = gacc;
        } else {
          facc[i][r] = __builtin_fmaf((float)gacc, st.s[t], facc[i][r]);
        }
      }
    }
  }
}

template <int TM, bool VEC, bool EXPORT, bool TILED>
__global__ __launch_bounds__(kW8Threads) void w4a8_mfma_kernel(GemmArgs a, int32_t *__restrict__ out) {
  constexpr int MB = 16 * TM;                         // activation rows per workgroup
  __shared__ __align__(16) float red[2][kW8Waves][TM][kWave][4];
  __shared__ __align__(16) int32_t as_lds[kW8Phase * MB];
  __shared__ __align__(16) float acc_lds[kW8Pass * MB * 16];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int q = lane >> 4, c = lane & 15;
  const int M = a.M, N = a.N, Kp = a.Kp, G = Kp / kGroup;
  const uint32_t rowbytes = (uint32_t)(Kp >> 1);
  const int m0 = blockIdx.y * MB;
  const int S = (N + 15) / 16;
  const int sb = (int)((long long)blockIdx.x * S / gridDim.x);
  const int se = (int)((long long)(blockIdx.x + 1) * S / gridDim.x);
  const int nph = (G + kW8Phase - 1) / kW8Phase;
  const int zadd = a.zeros ? 0 : 8;

  // row-major activations: this workgroup's rows, rows past M read 0.
  // tiled activations (w4a8_tiled_offset): all row blocks, blocks past the last read 0.
  const int mblocks = (M + 15) / 16;
  const Rsrc rx = TILED ? make_rsrc(a.xq, (uint32_t)(mblocks * 16 * Kp))
                        : make_rsrc(a.xq + (size_t)m0 * Kp, (uint32_t)(min(M - m0, MB) * Kp));
  const Rsrc ra = TILED ? make_rsrc(a.asum, (uint32_t)(mblocks * G * 16 * 4))
                        : make_rsrc(a.asum + (size_t)m0 * G, (uint32_t)(min(M - m0, MB) * G * 4));
  const Rsrc rw = make_rsrc(a.qw, (uint32_t)min((size_t)N * rowbytes, (size_t)0xFFFFFFF0u));
  const Rsrc rs = make_rsrc(a.scales, (uint32_t)((size_t)N * G * 4));
  const Rsrc rz = make_rsrc(a.zeros ? a.zeros : a.qw, a.zeros ? (uint32_t)(((size_t)N * G + 3) & ~(size_t)3) : 0u);

  // reduction role: thread -> (lane rl of the wave tiles, row block ri, row pair rp);
  // it sums two outputs of the 16*TM x 16 subtile over the waves
  const bool red_thread = threadIdx.x < TM * 2 * kWave;
  const int rl = threadIdx.x % kWave, ri = (threadIdx.x / kWave) >> 1, rp = (threadIdx.x / kWave) & 1;
  const int lr = 16 * ri + 4 * (rl >> 4) + 2 * rp;  // local row of the first output
  float xs0 = 0.f, xs1 = 0.f;
  if constexpr (!EXPORT) {
    // rows past M read 0 (their outputs are not stored)
    const Rsrc rxs = make_rsrc(a.xs + m0, (uint32_t)(min(M - m0, MB) * 4));
    xs0 = ld_f32(rxs, (uint32_t)lr * 4u);
    xs1 = ld_f32(rxs, (uint32_t)(lr + 1) * 4u);
  }

  v4i xlo[kW8GW][TM], xhi[kW8GW][TM];
  int buf = 0;
  const int pass_len = nph == 1 ? (se - sb) : kW8Pass;
  for (int p0 = sb; p0 < se; p0 += pass_len) {
    const int p1 = min(p0 + pass_len, se);
    for (int ph = 0; ph < nph; ph++) {
      const int gp = ph * kW8Phase;                    // first group of the phase
      const int gl0 = wave * kW8GW;                     // first group of this wave, within the phase
      const int gb = gp + gl0;
      const int gcnt = max(0, min(kW8GW, G - gb));
      // weights of the first subtile go out before the activations
      W8Stage sa, sbuf;
      w8_load<VEC>(sa, rw, rs, rz, 16 * p0 + c, N, gb, gcnt, G, rowbytes, q);
      if (nph > 1 || p0 == sb) {
#pragma unroll
        for (int t = 0; t < kW8GW; t++)
#pragma unroll
          for (int i = 0; i < TM; i++) {
            const bool ok = t < gcnt;
            uint32_t off, hstep;
            if constexpr (TILED) {
              off = (uint32_t)((((blockIdx.y * TM + i) * G + gb + t) * 2 * kWave + lane) * 16);
              hstep = kWave * 16;
            } else {
              off = (uint32_t)((16 * i + c) * Kp + (gb + t) * kGroup + 16 * q);
              hstep = 64;
            }
            xlo[t][i] = __builtin_bit_cast(v4i, ld_b128(rx, ok ? off : 0xFFFFFFF0u));
            xhi[t][i] = __builtin_bit_cast(v4i, ld_b128(rx, ok ? off + hstep : 0xFFFFFFF0u));
          }
        // group sums of the phase: all loads in flight together, then to LDS
        constexpr int APT = kW8Phase * MB / kW8Threads;
        int32_t av[APT];
#pragma unroll
        for (int k = 0; k < APT; k++) {
          const int e = threadIdx.x + k * kW8Threads;
          const int gl = e / MB, row = e % MB, m = m0 + row, g = gp + gl;
          uint32_t off;
          if constexpr (TILED)
            off = (uint32_t)(((blockIdx.y * TM + row / 16) * G + g) * 16 + row % 16) * 4u;
          else
            off = (uint32_t)((m - m0) * G + g) * 4u;
          av[k] = (int32_t)ld_u32(ra, (m < M && g < G) ? off : 0xFFFFFFF0u);
        }
        __syncthreads();  // as_lds of the previous phase is no longer read
#pragma unroll
        for (int k = 0; k < APT; k++) as_lds[threadIdx.x + k * kW8Threads] = av[k];
        __syncthreads();
      }
      for (int s = p0; s < p1; s += 2) {
        // subtile s from sa (prefetch s + 1 into sbuf), then s + 1 from sbuf (prefetch
        // s + 2 into sa). The prefetch is issued even past the range (as zero-length
        // reads), so that every path has the same loads in flight.
#pragma unroll
        for (int half = 0; half < 2; half++) {
          const int si = s + half;
          if (si >= p1) break;
          W8Stage &cur = half ? sbuf : sa;
          W8Stage &nxt = half ? sa : sbuf;
          w8_load<VEC>(nxt, rw, rs, rz, si + 1 < p1 ? 16 * (si + 1) + c : N, N, gb, gcnt, G, rowbytes, q);
          const int n = 16 * si + c;
          v4f facc[TM];
#pragma unroll
          for (int i = 0; i < TM; i++) facc[i] = v4f{0.f, 0.f, 0.f, 0.f};
          w8_compute<TM, VEC, EXPORT>(cur, xlo, xhi, as_lds, gl0, gcnt, zadd, facc, q, c, m0, M, n, N, G, gb, out);
          if constexpr (!EXPORT) {
#pragma unroll
            for (int i = 0; i < TM; i++) *reinterpret_cast<v4f *>(&red[buf][wave][i][lane][0]) = facc[i];
            __syncthreads();
            if (red_thread) {
              float v0 = 0.f, v1 = 0.f;
#pragma unroll
              for (int w = 0; w < kW8Waves; w++) {
                const v2f t = *reinterpret_cast<const v2f *>(&red[buf][w][ri][rl][2 * rp]);
                v0 += t.x;
                v1 += t.y;
              }
              const int nn = 16 * si + (rl & 15);
              float *acc_slot = acc_lds + ((si - p0) * MB + lr) * 16 + (rl & 15);
              if (ph > 0) {
                v0 = acc_slot[0] + v0;
                v1 = acc_slot[16] + v1;
              }
              if (ph + 1 < nph) {
                acc_slot[0] = v0;
                acc_slot[16] = v1;
              } else if (nn < N) {
                if (m0 + lr < M) a.y[(size_t)(m0 + lr) * N + nn] = v0 * xs0;
                if (m0 + lr + 1 < M) a.y[(size_t)(m0 + lr + 1) * N + nn] = v1 * xs1;
              }
            }
            buf ^= 1;
          }
        }
      }
    }
  }
}

// ------------------------------------------------------------ W4A8 GEMM (int8 MFMA), Y only
//
// The kernel above also serves the exact group-accumulator export; this one only
// produces Y and is arranged around the three limits of the batch regime:
//   * VALU: per (16x16 tile, group) the int32 accumulator of the raw codes needs a
//     conversion and one FMA with the group scale (8 VALU for 2 MFMA). The
//     zero-point term is not subtracted per group: since
//       sum_g s_g (sum_k q a - z_g asum_g) = sum_g s_g sum_k q a - sum_g (s_g z_g) asum_g,
//     the second sum over a wave's four groups is one v_mfma_f32_16x16x4_f32 per
//     row block (A = asum of the 16 rows x 4 groups, B = -s z of the 16 weight rows
//     x 4 groups), accumulated into the same fp32 tile.
//   * latency: a workgroup's subtiles form one chunk (up to NS), whose weight loads
//     are all in flight (PF stages ahead of the one computed): each subtile's
//     partial tile goes to the LDS reduction buffer as it completes, so registers
//     hold weights rather than accumulators, and the waves' tiles are reduced once
//     per chunk with one barrier. Loads are issued in need order (first subtile,
//     activations, later subtiles) behind scheduling barriers, and every load is
//     unconditional, so each subtile waits for its own stage alone.
//   * L1/L2 bandwidth: every workgroup reads its 16*TM activation rows once per
//     K phase into registers; TM is chosen per shape to minimise the bytes each CU
//     must read (activations + its share of the weights).
// Waves split the K groups as in the kernel above (wave w: groups 4w..4w+3 of each
// phase of 32). fp32 rounding of the split terms stays within the reference's W4A8
// bound, which is built from both magnitudes (sum q|a| and z|sum a|).

constexpr int kW8GB = 1;  // groups whose MFMAs are issued together

// Weight operands of one subtile when all four of the wave's groups exist and G % 4
// == 0 (or the weights are in the t16 layout): four 16-byte loads from one offset
// register (group offsets are immediates), the four scales as one 16-byte load and
// the four zero-points as one dword. Rows past N start past the end of their
// descriptors and read 0.
template <bool WT>
__device__ __forceinline__ void w8_load_full(W8Stage &st, Rsrc rw, Rsrc rs, Rsrc rz, uint32_t woff, uint32_t goff) {
#pragma unroll
  for (int t = 0; t < kW8GW; t++) st.w[t] = ld_b128(rw, woff + (WT ? 1024u : 64u) * t);
  const float4 sv = ld_f4(rs, goff * 4u);
  st.s[0] = sv.x;
  st.s[1] = sv.y;
  st.s[2] = sv.z;
  st.s[3] = sv.w;
  st.zw[0] = ld_u32(rz, goff);
}

// One 16-row weight subtile against the wave's activation operands: the zero-point
// MFMA first (its result is needed only by the FMAs at the end), then all first
// MFMAs (low nibbles), all second MFMAs (high nibbles, accumulating onto the first:
// they issue 4*TM MFMAs after their operand, past its latency), then the fp32
// rescale of every group accumulator.
template <int TM>
__device__ __forceinline__ void w8_tile(const W8Stage &cur, const v4i (&xlo)[kW8GW][TM], const v4i (&xhi)[kW8GW][TM],
                                        const float (&asf)[TM], float bz, v4f (&facc)[TM]) {
#pragma unroll
  for (int i = 0; i < TM; i++) facc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(asf[i], bz, facc[i], 0, 0, 0);
  // groups in batches of kW8GB: all low-nibble MFMAs of the batch, then all
  // high-nibble ones, then the rescale
  const v4i zero4 = {0, 0, 0, 0};
#pragma unroll
  for (int t0 = 0; t0 < kW8GW; t0 += kW8GB) {
    v4i bhi[kW8GB], acc[kW8GB][TM];
#pragma unroll
    for (int u = 0; u < kW8GB; u++) {
      const uint4 w = cur.w[t0 + u];
      const v4i blo = {(int)lo_nibbles(w.x), (int)lo_nibbles(w.y), (int)lo_nibbles(w.z), (int)lo_nibbles(w.w)};
      bhi[u] = v4i{(int)hi_nibbles(w.x), (int)hi_nibbles(w.y), (int)hi_nibbles(w.z), (int)hi_nibbles(w.w)};
#pragma unroll
      for (int i = 0; i < TM; i++) acc[u][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xlo[t0 + u][i], blo, zero4, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kW8GB; u++)
#pragma unroll
      for (int i = 0; i < TM; i++)
        acc[u][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xhi[t0 + u][i], bhi[u], acc[u][i], 0, 0, 0);
#pragma unroll
    for (int u = 0; u < kW8GB; u++)
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) facc[i][r] = __builtin_fmaf((float)acc[u][i][r], cur.s[t0 + u], facc[i][r]);
  }
}

// FULL (G % 32 == 0): every wave has all four groups in every phase, so the weight
// loads take the vector path with no per-group clamps.
// WT: weights in the t16 tile layout, so each 16-byte weight load of a wave is one
// contiguous 1 KiB tile instead of 64 bytes from each of 16 rows (the row-major
// pattern runs at about half the cache bandwidth). Groups past G hold zeros there.
template <int TM, int NS, int PF, bool VEC, bool FULL, bool TILED, bool WT>
__global__ __launch_bounds__(kW8Threads) void w4a8_gemm_kernel(GemmArgs a) {
  static_assert(!FULL || VEC, "the full path needs G % 4 == 0");
  static_assert(!WT || VEC, "the t16 layout pads groups to a multiple of 4");
  // partial tiles of every wave: [NS][TM][wave][lane] x 4 floats
  __shared__ __align__(16) float red[NS * TM * kW8Waves * kWave * 4];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int q = lane >> 4, c = lane & 15;
  const int M = a.M, N = a.N, Kp = a.Kp, G = Kp / kGroup;
  const uint32_t rowbytes = (uint32_t)(Kp >> 1);
  constexpr int MB = 16 * TM;
  const int mb0 = blockIdx.y * TM, m0 = mb0 * 16;
  const int S = (N + 15) / 16;
  // subtiles [sb, se): S / gridDim.x each, one more for the first S % gridDim.x
  const int sbase = (int)((unsigned)S / gridDim.x), srem = S - sbase * (int)gridDim.x;
  const int bx = blockIdx.x;
  const int sb = bx * sbase + min(bx, srem), se = sb + sbase + (bx < srem ? 1 : 0);
  const int nph = (G + kW8Phase - 1) / kW8Phase;
  const int zadd = a.zeros ? 0 : 8;

  const int mblocks = (M + 15) / 16;
  const Rsrc rx = TILED ? make_rsrc(a.xq, (uint32_t)(mblocks * 16 * Kp))
                        : make_rsrc(a.xq + (size_t)m0 * Kp, (uint32_t)(min(M - m0, MB) * Kp));
  const Rsrc ra = TILED ? make_rsrc(a.asum, (uint32_t)(mblocks * G * 16 * 4))
                        : make_rsrc(a.asum + (size_t)m0 * G, (uint32_t)(min(M - m0, MB) * G * 4));
  const int G4 = (G + 3) & ~3;  // groups per subtile in the t16 layout
  const size_t wbytes = WT ? t16_qw_bytes(N, Kp) : (size_t)N * rowbytes;
  const size_t gents = WT ? t16_group_entries(N, Kp) : (size_t)N * G;
  const Rsrc rw = make_rsrc(a.qw, (uint32_t)min(wbytes, (size_t)0xFFFFFFF0u));
  const Rsrc rs = make_rsrc(a.scales, (uint32_t)(gents * 4));
  const Rsrc rz = make_rsrc(a.zeros ? a.zeros : a.qw, a.zeros ? (uint32_t)((gents + 3) & ~(size_t)3) : 0u);
  const Rsrc rxs = make_rsrc(a.xs + m0, (uint32_t)(min(M - m0, MB) * 4));

  // per-token scales of the four rows this thread stores in the reduction: its
  // lane l = threadIdx.x % 64 and row block i = (threadIdx.x / 64) % TM are the same
  // for every item it takes (512 is a multiple of 64 * TM); loaded up front
  // because a wait for a load issued after the Y stores would wait for them too
  static_assert(kW8Waves % TM == 0, "each thread must keep one row block in the reduction");
  const int rlane = threadIdx.x & (kWave - 1), rblk = (threadIdx.x / kWave) % TM;
  const int rrow = 16 * rblk + 4 * (rlane >> 4);  // local row of the thread's first output
  // one dword per row: a 16-byte load straddling the end of the rows would read 0
  float xsr[4];
#pragma unroll
  for (int r = 0; r < 4; r++) xsr[r] = ld_f32(rxs, (uint32_t)(rrow + r) * 4u);

  v4i xlo[kW8GW][TM], xhi[kW8GW][TM];
  float asf[TM];
  // partial tiles: in registers across the phases of a chunk for the tall tiles
  // (TM = 4: their activations fill half the register file), otherwise written
  // to the LDS reduction buffer as each subtile completes, which frees the
  // registers for more weight subtiles in flight
  constexpr bool kRegAcc = TM >= 4;
  for (int cb = sb; cb < se; cb += NS) {
    const int ce = min(cb + NS, se);
    v4f racc[kRegAcc ? NS : 1][TM];
    if constexpr (kRegAcc) {
#pragma unroll
      for (int j = 0; j < NS; j++)
#pragma unroll
        for (int i = 0; i < TM; i++) racc[j][i] = v4f{0.f, 0.f, 0.f, 0.f};
    }
    for (int ph = 0; ph < nph; ph++) {
      const int gb = ph * kW8Phase + wave * kW8GW;     // this wave's first group
      const int gcnt = max(0, min(kW8GW, G - gb));
      // row-major: row n of subtile s has its weights at n * rowbytes + gb * 64 + q * 16
      // and its group data at n * G + gb; t16: tile (s, gb + t) at ((s G4 + gb + t) 64 +
      // lane) 16 and the four groups' data at ((s G4/4 + gb/4) 16 + c) 4
      const uint32_t wstep = WT ? (uint32_t)G4 * 1024u : 16u * rowbytes;
      const uint32_t gstep = WT ? (uint32_t)G4 * 16u : 16u * (uint32_t)G;
      const uint32_t woff0 = WT ? ((uint32_t)cb * G4 + gb) * 1024u + (uint32_t)lane * 16u
                                : (uint32_t)(16 * cb + c) * rowbytes + (uint32_t)gb * 64u + (uint32_t)q * 16u;
      const uint32_t goff0 = WT ? ((uint32_t)cb * (G4 / 4) + gb / 4) * 64u + (uint32_t)c * 4u
                                : (uint32_t)(16 * cb + c) * (uint32_t)G + (uint32_t)gb;
      auto load = [&](W8Stage &st, int j) {
        const int sj = cb + j;
        const bool in = j < NS && sj < ce;  // past the chunk: rows past N, zero-length reads
        if constexpr (FULL || WT) {
          // past the matrix: subtile S + 1 starts beyond every descriptor
          const uint32_t jj = in ? (uint32_t)j : (uint32_t)(S - cb + 1);
          w8_load_full<WT>(st, rw, rs, rz, woff0 + jj * wstep, goff0 + jj * gstep);
        } else {
          w8_load<VEC>(st, rw, rs, rz, in ? 16 * sj + c : N, N, gb, gcnt, G, rowbytes, q);
        }
      };
      // issue order = retirement order: the first subtile's weights, then the
      // activations, then the other PF subtiles of the chunk, so the first
      // MFMAs wait for the first subtile and the activations alone. Every load
      // is unconditional (stages past the chunk read zero-length ranges, and a
      // later chunk reloads the activations from the cache) so that the compiler
      // can count the loads in flight and wait for exactly the ones needed. The
      // tall tiles take one subtile per chunk, many chunks per workgroup: they
      // load the activations once per phase (their waits are for whole chunks)
      W8Stage st[PF + 1];
      load(st[0], 0);
      if (!kRegAcc || nph > 1 || cb == sb) {
        // activation operands of this wave's groups (groups past G read 0, so the
        // weights of those slots never matter) and the group sums of the
        // zero-point MFMA (lane (q, c): row c of the block, group gb + q)
#pragma unroll
        for (int t = 0; t < kW8GW; t++)
#pragma unroll
          for (int i = 0; i < TM; i++) {
            const bool ok = t < gcnt;
            uint32_t off, hstep;
            if constexpr (TILED) {
              off = (uint32_t)((((mb0 + i) * G + gb + t) * 2 * kWave + lane) * 16);
              hstep = kWave * 16;
            } else {
              off = (uint32_t)((16 * i + c) * Kp + (gb + t) * kGroup + 16 * q);
              hstep = 64;
            }
            xlo[t][i] = __builtin_bit_cast(v4i, ld_b128(rx, ok ? off : 0xFFFFFFF0u));
            xhi[t][i] = __builtin_bit_cast(v4i, ld_b128(rx, ok ? off + hstep : 0xFFFFFFF0u));
          }
#pragma unroll
        for (int i = 0; i < TM; i++) {
          uint32_t off;
          if constexpr (TILED)
            off = (uint32_t)((((mb0 + i) * G + gb + q) * 16 + c) * 4);
          else
            off = (uint32_t)(((16 * i + c) * G + gb + q) * 4);
          asf[i] = (float)(int32_t)ld_u32(ra, q < gcnt ? off : 0xFFFFFFF0u);
        }
      }
      // the scheduler would otherwise group the loads by type, moving each
      // subtile's scales behind every later weight load
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 1; j <= PF; j++) {
        load(st[j], j);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int j = 0; j < NS; j++) {
        if (cb + j >= ce) break;  // workgroup-uniform
        W8Stage &cur = st[j % (PF + 1)];
        const int n = 16 * (cb + j) + c;
        if constexpr (!FULL) {
          // groups past G: zero scales (their activations are zero too)
#pragma unroll
          for (int t = 0; t < kW8GW; t++) cur.s[t] = t < gcnt ? cur.s[t] : 0.0f;
        }
        // -s * z of group gb + q for weight row n: B operand of the zero-point MFMA
        float sq = cur.s[0];
        sq = q == 1 ? cur.s[1] : sq;
        sq = q == 2 ? cur.s[2] : sq;
        sq = q == 3 ? cur.s[3] : sq;
        int zq;
        if constexpr (VEC) {
          zq = (int)((cur.zw[0] >> (8 * q)) & 0xFFu);
        } else {
          const int z0 = w8_zero<VEC>(cur, 0, n, G, gb), z1 = w8_zero<VEC>(cur, 1, n, G, gb),
                    z2 = w8_zero<VEC>(cur, 2, n, G, gb), z3 = w8_zero<VEC>(cur, 3, n, G, gb);
          zq = q == 1 ? z1 : z0;
          zq = q == 2 ? z2 : zq;
          zq = q == 3 ? z3 : zq;
        }
        const float bz = -sq * (float)(zq + zadd);
        if constexpr (kRegAcc) {
          w8_tile<TM>(cur, xlo, xhi, asf, bz, racc[j]);
        } else {
          // each thread owns its LDS slots, so no barrier is needed until the
          // reduction; later phases add onto the earlier ones
          v4f *slot = reinterpret_cast<v4f *>(&red[((j * TM * kW8Waves + wave) * kWave + lane) * 4]);
          v4f facc[TM];
#pragma unroll
          for (int i = 0; i < TM; i++) facc[i] = v4f{0.f, 0.f, 0.f, 0.f};
          w8_tile<TM>(cur, xlo, xhi, asf, bz, facc);
          if (ph == 0) {
#pragma unroll
            for (int i = 0; i < TM; i++) slot[i * kW8Waves * kWave] = facc[i];
          } else {
#pragma unroll
            for (int i = 0; i < TM; i++) slot[i * kW8Waves * kWave] += facc[i];
          }
        }
        // refill this stage with subtile j + PF + 1 (zero-length past the chunk)
        if (j + PF + 1 < NS) load(cur, j + PF + 1);
      }
    }
    // ---- reduce the waves' partial tiles of the chunk, scale by xs, store
    if constexpr (kRegAcc) {
#pragma unroll
      for (int j = 0; j < NS; j++)
#pragma unroll
        for (int i = 0; i < TM; i++)
          *reinterpret_cast<v4f *>(&red[(((j * TM + i) * kW8Waves + wave) * kWave + lane) * 4]) = racc[j][i];
    }
    __syncthreads();
    for (int e = threadIdx.x; e < (ce - cb) * TM * kWave; e += kW8Threads) {
      const int j = e / (kWave * TM);  // e % 64 == rlane, (e / 64) % TM == rblk
      v4f v = *reinterpret_cast<const v4f *>(&red[(((j * TM + rblk) * kW8Waves + 0) * kWave + rlane) * 4]);
#pragma unroll
      for (int w = 1; w < kW8Waves; w++) {
        const v4f t = *reinterpret_cast<const v4f *>(&red[(((j * TM + rblk) * kW8Waves + w) * kWave + rlane) * 4]);
        v += t;
      }
      const int n = 16 * (cb + j) + (rlane & 15);
      if (n < N) {
#pragma unroll
        for (int r = 0; r < 4; r++)
          if (m0 + rrow + r < M) a.y[(size_t)(m0 + rrow + r) * N + n] = v[r] * xsr[r];
      }
    }
    __syncthreads();  // red is rewritten by the next chunk
  }
}

// Subtiles per chunk (NS: their partial tiles share the LDS reduction buffer) and
// weight subtiles in flight ahead of the one computed (PF: PF + 1 stages of
// registers next to the 2 * TM * kW8GW activation operands; PF for t16 weights,
// PFR for row-major ones and PFS for the per-group weight loads of G % 4 != 0,
// whose addressing needs more registers). PFR and PFS are the largest values that
// compile without spills; PF is not: with t16 weights, deeper prefetch queues so
// many weight loads ahead of the activation operands that the first tile starts
// later (per-wave timelines at 64 x 11008 x 4096: first tile 5.6 us after the start
// with 5 subtiles in flight, 3.4 us with 2; the GEMM 10.5 -> 8.5 us). Two 16-row
// blocks (TM = 2) keep one subtile in flight: 160 VGPRs instead of 182, and the
// quantizer + GEMM call at 64 x 11008 x 4096 hot 12.42-12.47 -> 12.05-12.10 us
// (alternating in one process; 64 x 4096 x 4096 within 0.1 us either way). More
// waves did not help: 16-row blocks at two workgroups per CU (4 waves per SIMD,
// 111-118 VGPRs) took 13.1-13.8 us.
template <int TM> struct W8Cfg {
  static constexpr int NS = TM >= 4 ? 1 : 6;
  static constexpr int PF = TM >= 4 ? 0 : TM == 2 ? 1 : 2;
  static constexpr int PFR = TM >= 4 ? 0 : 4;
  static constexpr int PFS = TM >= 4 ? 0 : TM == 2 ? 2 : 3;
};

// Calls go(std::integral_constant<int, P>) with the stages in flight a workgroup
// of spw subtiles needs: every load is issued, so stages past the workgroup's
// subtiles would only cost issue slots (0 for one subtile, 1 for two, 3 for up
// to four, else PFMAX).
template <int PFMAX, typename Go>
static void with_prefetch(int spw, Go &&go) {
  if constexpr (PFMAX == 0) {
    go(std::integral_constant<int, 0>{});
  } else {
    if (spw <= 1) go(std::integral_constant<int, 0>{});
    else if (spw <= 2) go(std::integral_constant<int, 1>{});
    else if (spw <= 4 || PFMAX <= 3) go(std::integral_constant<int, (PFMAX < 3 ? PFMAX : 3)>{});
    else go(std::integral_constant<int, PFMAX>{});
  }
}

template <int TM, bool TILED>
static void launch_w4a8_gemm_t(const GemmArgs &a, dim3 grid, hipStream_t s) {
  constexpr int NS = W8Cfg<TM>::NS, PF = W8Cfg<TM>::PF, PFR = W8Cfg<TM>::PFR, PFS = W8Cfg<TM>::PFS;
  const int G = a.Kp / kGroup;
  const int spw = ((a.N + 15) / 16 + (int)grid.x - 1) / (int)grid.x;  // subtiles per workgroup
  if (a.wt16) {
    with_prefetch<PF>(spw, [&](auto pf) {
      constexpr int P = decltype(pf)::value;
      if (G % kW8Phase == 0)
        hipLaunchKernelGGL((w4a8_gemm_kernel<TM, NS, P, true, true, true, true>), grid, dim3(kW8Threads), 0, s, a);
      else
        hipLaunchKernelGGL((w4a8_gemm_kernel<TM, NS, P, true, false, true, true>), grid, dim3(kW8Threads), 0, s, a);
    });
  } else if (G % kW8Phase == 0) {
    hipLaunchKernelGGL((w4a8_gemm_kernel<TM, NS, PFR, true, true, TILED, false>), grid, dim3(kW8Threads), 0, s, a);
  } else if (G % 4 == 0) {
    hipLaunchKernelGGL((w4a8_gemm_kernel<TM, NS, PFR, true, false, TILED, false>), grid, dim3(kW8Threads), 0, s, a);
  } else {
    hipLaunchKernelGGL((w4a8_gemm_kernel<TM, NS, PFS, false, false, TILED, false>), grid, dim3(kW8Threads), 0, s, a);
  }
}

// Per-CU bytes of the (TM) tiling: the workgroup's activation rows plus its share
// of the weights, with one workgroup per CU.
static double w4a8_cu_bytes(int tm, int M, int N, int Kp, int cus, int &gx) {
  const int gy = (M + 16 * tm - 1) / (16 * tm);
  const int S = (N + 15) / 16;
  gx = std::max(1, std::min(S, cus / gy));
  const double spw = (double)((S + gx - 1) / gx);
  const double wrow = Kp / 2 + (Kp / kGroup) * 5.0;
  return (double)tm * 16 * Kp + spw * 16 * wrow;
}

static hipError_t launch_w4a8_gemm(const GemmArgs &a, int num_cus, hipStream_t s) {
  const int cus = num_cus > 0 ? num_cus : 256;
  const int mb = (a.M + 15) / 16;
  int best_tm = 1, best_gx = 1;
  double best = 1e300;
  for (int tm : {1, 2, 4}) {
    if (tm > 1 && tm > mb) break;  // no taller tile than the row blocks there are
    int gx;
    const double b = w4a8_cu_bytes(tm, a.M, a.N, a.Kp, cus, gx);
    if (b < best * 0.97) best = b, best_tm = tm, best_gx = gx;
  }
  const dim3 grid(best_gx, (a.M + 16 * best_tm - 1) / (16 * best_tm));
  if (a.wt16 && !a.tiled) return hipErrorInvalidValue;  // the t16 path reads tiled activations
  if (a.tiled) {
    if (best_tm == 1) launch_w4a8_gemm_t<1, true>(a, grid, s);
    else if (best_tm == 2) launch_w4a8_gemm_t<2, true>(a, grid, s);
    else launch_w4a8_gemm_t<4, true>(a, grid, s);
  } else {
    if (best_tm == 1) launch_w4a8_gemm_t<1, false>(a, grid, s);
    else if (best_tm == 2) launch_w4a8_gemm_t<2, false>(a, grid, s);
    else launch_w4a8_gemm_t<4, false>(a, grid, s);
  }
  return hipGetLastError();
}

template <int TM, bool EXPORT, bool TILED>
static void launch_w4a8_v(const GemmArgs &a, int32_t *out, dim3 grid, hipStream_t s) {
  if ((a.Kp / kGroup) % 4 == 0)
    hipLaunchKernelGGL((w4a8_mfma_kernel<TM, true, EXPORT, TILED>), grid, dim3(kW8Threads), 0, s, a, out);
  else
    hipLaunchKernelGGL((w4a8_mfma_kernel<TM, false, EXPORT, TILED>), grid, dim3(kW8Threads), 0, s, a, out);
}

template <int TM>
static hipError_t launch_w4a8_tm(const GemmArgs &a, int32_t *out, int num_cus, hipStream_t s) {
  const int S = (a.N + 15) / 16;
  const int per_cu = TM == 1 ? 2 : 1;  // workgroups resident per CU (VGPR budget)
  const int cus = num_cus > 0 ? num_cus : 256;
  const int gx = S < per_cu * cus ? S : per_cu * cus;
  dim3 grid(gx, (a.M + 16 * TM - 1) / (16 * TM));
  if (out)
    launch_w4a8_v<TM, true, false>(a, out, grid, s);
  else if (a.tiled)
    launch_w4a8_v<TM, false, true>(a, out, grid, s);
  else
    launch_w4a8_v<TM, false, false>(a, out, grid, s);
  return hipGetLastError();
}

hipError_t launch_w4a8_mfma(const GemmArgs &a, int32_t *out, int num_cus, hipStream_t s) {
  if (!out) return launch_w4a8_gemm(a, num_cus, s);
  if (a.M <= 16) return launch_w4a8_tm<1>(a, out, num_cus, s);
  if (a.M <= 32) return launch_w4a8_tm<2>(a, out, num_cus, s);
  if (a.M <= 48) return launch_w4a8_tm<3>(a, out, num_cus, s);
  return launch_w4a8_tm<4>(a, out, num_cus, s);
}

// ============================================================ W4A16 / MXFP4, bf16x3 MFMA
//
// fp32 semantics on bf16 matrix cores. Each activation is split into three bf16
// terms, x = hi + mid + lo exactly; each weight is exact in bf16 (W4A16: the integer
// q - z in [-15, 15]; MXFP4: E2M1 times a power of two). Every product of
// v_mfma_f32_16x16x32_bf16 is therefore an exact float32 value and the sums are
// float32, as in the reference's fp32 kernels; three bf16 MFMAs per product run at
// 16x the fp32 MFMA rate each (2.5 PFLOP/s against 157 TFLOP/s dense).
//
// Operand slots (lane l = 16q + c, 8 bf16 per operand, slot s = 0..7, u = 0..3 the
// four 32-wide MFMAs of a 128-element group g); A and B agree slot by slot:
//   W4A16: weight bytes [64g + 16q, +16) of row c (t16 tile): u = 0/1 low nibbles of
//          bytes 0-7 / 8-15, u = 2/3 high nibbles; element 128g + 64 (u>>1) + 16q +
//          8 (u&1) + s.
//   MXFP4: the lane's 16 bytes are block b = 4g + q; u takes bytes 4u .. 4u+3, each
//          byte giving (low, high) nibble = elements (32b + j, 32b + 16 + j): slot s
//          is element 32b + 4u + (s>>1) + 16 (s&1).
// The split activations are tiled [row block][group][u][term][lane][16 B], so a
// wave reads every operand with one contiguous 1 KiB load.

template <int F>
__global__ __launch_bounds__(kThreads) void split3_kernel(const float *__restrict__ x, int M, int Kp,
                                                          uint4 *__restrict__ x3) {
  const int G = (Kp + 127) / 128, mblocks = (M + 15) / 16;
  const size_t total = (size_t)mblocks * G * 4 * kWave;
  const Rsrc rx = make_rsrc(x, (uint32_t)((size_t)M * Kp * 4));
  for (size_t t = (size_t)blockIdx.x * kThreads + threadIdx.x; t < total; t += (size_t)gridDim.x * kThreads) {
    const int lane = (int)(t % kWave), u = (int)((t / kWave) % 4);
    const size_t gi = t / (4 * kWave);  // row block * G + group
    const int g = (int)(gi % G), mb = (int)(gi / G);
    const int row = 16 * mb + (lane & 15), q = lane >> 4;
    float v[8];
    if constexpr (F == F_W4A16) {
      const int e0 = 128 * g + 64 * (u >> 1) + 16 * q + 8 * (u & 1);
      const bool ok = row < M;  // Kp % 128 == 0
      const uint32_t off = (uint32_t)(((size_t)row * Kp + e0) * 4);
      const float4 lo = ld_f4(rx, ok ? off : 0xFFFFFFF0u), hi = ld_f4(rx, ok ? off + 16 : 0xFFFFFFF0u);
      v[0] = lo.x; v[1] = lo.y; v[2] = lo.z; v[3] = lo.w;
      v[4] = hi.x; v[5] = hi.y; v[6] = hi.z; v[7] = hi.w;
    } else {
      const int b = 4 * g + q, e0 = 32 * b + 4 * u;
      const bool ok = row < M && 32 * b < Kp;
      const uint32_t off = (uint32_t)(((size_t)row * Kp + e0) * 4);
      const float4 lo = ld_f4(rx, ok ? off : 0xFFFFFFF0u), hi = ld_f4(rx, ok ? off + 64 : 0xFFFFFFF0u);
      v[0] = lo.x; v[1] = hi.x; v[2] = lo.y; v[3] = hi.y;
      v[4] = lo.z; v[5] = hi.z; v[6] = lo.w; v[7] = hi.w;
    }
    uint32_t th[8], tm[8], tl[8];
#pragma unroll
    for (int k = 0; k < 8; k++) split3(v[k], th[k], tm[k], tl[k]);
    uint4 *dst = x3 + (gi * 4 + u) * 3 * kWave + lane;
    dst[0] = make_uint4(pack_bf16(th[0], th[1]), pack_bf16(th[2], th[3]), pack_bf16(th[4], th[5]), pack_bf16(th[6], th[7]));
    dst[kWave] = make_uint4(pack_bf16(tm[0], tm[1]), pack_bf16(tm[2], tm[3]), pack_bf16(tm[4], tm[5]), pack_bf16(tm[6], tm[7]));
    dst[2 * kWave] = make_uint4(pack_bf16(tl[0], tl[1]), pack_bf16(tl[2], tl[3]), pack_bf16(tl[4], tl[5]), pack_bf16(tl[6], tl[7]));
  }
}

hipError_t launch_split3(int fmt, const float *x, int M, int Kp, uint4 *x3, hipStream_t s) {
  const size_t work = (size_t)((M + 15) / 16) * ((Kp + 127) / 128) * 4 * kWave;
  size_t blocks = (work + kThreads - 1) / kThreads;
  if (blocks > 16384) blocks = 16384;
  if (fmt == F_W4A16)
    hipLaunchKernelGGL(split3_kernel<F_W4A16>, dim3((unsigned)blocks), dim3(kThreads), 0, s, x, M, Kp, x3);
  else
    hipLaunchKernelGGL(split3_kernel<F_MXFP4>, dim3((unsigned)blocks), dim3(kThreads), 0, s, x, M, Kp, x3);
  return hipGetLastError();
}

// W4A16 activations as two float16 terms for the f16 matrix cores (one workgroup per
// row). The row is scaled by 2^E, E chosen so that its largest magnitude lands in
// [2^14, 2^15) (E = 0 for a zero or non-finite row); then xs = x 2^E = hi + lo 2^-11
// with hi = fp16(xs) and lo = fp16((xs - hi) 2^11) (the remainder is exact in fp32;
// the 2^11 keeps lo clear of float16's subnormals, which the matrix cores flush, for
// |xs| >= 2^-3). So an element keeps 22 significant bits within 2^17 of the row's
// largest, has an absolute error of at most 2^-39 of the largest down to 2^28 below
// it, and is dropped below that. Slots as in split3_kernel's W4A16 tiles, two terms
// per slot.
// Workgroups (m, p) of a row each take the row's maximum over all of it (from the
// caches after the first) and split part p of its slots.
__global__ __launch_bounds__(kThreads) void split2h_kernel(const float *__restrict__ x, int M, int Kp,
                                                          uint4 *__restrict__ x2, int *__restrict__ xexp) {
  __shared__ float red[kThreads / kWave];
  const int m = blockIdx.x, G = Kp / 128, items = G * 16;  // (g, u, q): 8 elements each
  const int P = gridDim.y, pt0 = (int)(((long long)items * blockIdx.y) / P),
            pt1 = (int)(((long long)items * (blockIdx.y + 1)) / P);
  const float *xr = x + (size_t)m * Kp;
  auto e0_of = [](int t) { return 128 * (t >> 4) + 64 * ((t >> 3) & 1) + 16 * (t & 3) + 8 * ((t >> 2) & 1); };
  float amax = 0.0f;
  for (int t = threadIdx.x; t < items; t += kThreads) {
    const float4 lo = *reinterpret_cast<const float4 *>(xr + e0_of(t));
    const float4 hi = *reinterpret_cast<const float4 *>(xr + e0_of(t) + 4);
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(lo.x), fabsf(lo.y)), fmaxf(fabsf(lo.z), fabsf(lo.w))));
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(hi.x), fabsf(hi.y)), fmaxf(fabsf(hi.z), fabsf(hi.w))));
  }
  amax = wave_max(amax);
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = amax;
  __syncthreads();
  float rmax = red[0];
#pragma unroll
  for (int w = 1; w < kThreads / kWave; w++) rmax = fmaxf(rmax, red[w]);
  int E = 0;
  if (rmax > 0.0f && rmax <= 3.402823466e38f) {
    int ex;
    frexpf(rmax, &ex);  // rmax = f 2^ex, f in [0.5, 1)
    E = 15 - ex;
  }
  if (threadIdx.x == 0 && blockIdx.y == 0) xexp[m] = E;
  const int mb = m >> 4, r = m & 15;
  for (int t = pt0 + (int)threadIdx.x; t < pt1; t += kThreads) {
    const float4 lo = *reinterpret_cast<const float4 *>(xr + e0_of(t));
    const float4 hi = *reinterpret_cast<const float4 *>(xr + e0_of(t) + 4);
    const float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    uint32_t th[4], tl[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const float a0 = ldexpf(v[2 * k], E), a1 = ldexpf(v[2 * k + 1], E);
      const _Float16 h0 = (_Float16)a0, h1 = (_Float16)a1;
      const _Float16 l0 = (_Float16)((a0 - (float)h0) * 2048.0f), l1 = (_Float16)((a1 - (float)h1) * 2048.0f);
      th[k] = __builtin_bit_cast(uint32_t, h2v{h0, h1});
      tl[k] = __builtin_bit_cast(uint32_t, h2v{l0, l1});
    }
    const int g = t >> 4, u = (t >> 2) & 3, q = t & 3;
    uint4 *dst = x2 + (((size_t)mb * G + g) * 4 + u) * 2 * kWave + 16 * q + r;
    dst[0] = make_uint4(th[0], th[1], th[2], th[3]);
    dst[kWave] = make_uint4(tl[0], tl[1], tl[2], tl[3]);
  }
}

hipError_t launch_split2h(const float *x, int M, int Kp, uint4 *x2, int *xexp, hipStream_t s) {
  if (M <= 0 || Kp % 128) return hipErrorInvalidValue;
  // about 256 workgroups: each row's slots in up to G parts
  const int G = Kp / 128, P = std::max(1, std::min(G, 256 / M));
  hipLaunchKernelGGL(split2h_kernel, dim3(M, P), dim3(kThreads), 0, s, x, M, Kp, x2, xexp);
  return hipGetLastError();
}

// Weight stage of one subtile: the lane's 16 bytes of the group's tile and, for
// W4A16, its row's scale and the dword of zero-points holding its group's; for
// MXFP4, the dword of E8M0 bytes holding its block's; for the t16f8 layout, the
// lane's 32 bytes (w, w2) and its row's scale. Bytes are extracted where they are
// used (a byte load's zero extension next to the load would make each stage wait
// for its own load).
struct B3Stage {
  uint4 w, w2;
  float s;
  uint32_t z;
};

// Four float32 of (byte k of nib) - zf as two bf16x2 (exact: integers below 16).
__device__ __forceinline__ void w4_bf16x4(uint32_t nib, float zf, uint32_t &d0, uint32_t &d1) {
  const uint32_t n = opaque(nib);
  const float f0 = (float)(n & 0xFF) - zf, f1 = (float)((n >> 8) & 0xFF) - zf;
  const float f2 = (float)((n >> 16) & 0xFF) - zf, f3 = (float)(n >> 24) - zf;
  d0 = pack_bf16(__float_as_uint(f0), __float_as_uint(f1));
  d1 = pack_bf16(__float_as_uint(f2), __float_as_uint(f3));
}

// Four float32 of (byte k of nib) - zf as two float16x2 (exact: integers below 16).
__device__ __forceinline__ void w4_f16x4(uint32_t nib, float zf, uint32_t &d0, uint32_t &d1) {
  const uint32_t n = opaque(nib);
  const float f0 = (float)(n & 0xFF) - zf, f1 = (float)((n >> 8) & 0xFF) - zf;
  const float f2 = (float)((n >> 16) & 0xFF) - zf, f3 = (float)(n >> 24) - zf;
  d0 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(f0, f1));
  d1 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(f2, f3));
}

// Waves split the K groups (wave w takes group 8 ph + w of phase ph) and keep
// their activation operands (4 x 3 x TM x 1 KiB) in registers across the
// workgroup's subtiles; per subtile and row block, 12 MFMAs accumulate the group
// (W4A16) or the four blocks (MXFP4) and one FMA per output applies the fp32
// factor. A chunk holds up to NS subtiles (normally all of the workgroup's), so
// each phase's activations are loaded once per workgroup; each subtile's partial
// tile is kept in the LDS reduction buffer (each thread owns its slots, later
// phases accumulate onto them), which leaves the registers for PF weight
// subtiles in flight. Partial tiles are reduced across waves in LDS once per
// chunk, in a fixed order.
// F8 (W4A16 only): the weights are in the t16f8 layout, each lane's 32 codes
// already less their zero-point as E4M3 bytes n 2^-9 (sign and magnitude n <= 15),
// so that one conversion with scale 2^9 makes two bf16 operands, the same values
// as the nibble path's (float)code - z, with no zero-point load.
// H2 (W4A16 only): the activations as two float16 terms of each row times 2^E
// (split2h_kernel) on the float16 matrix cores, 8 MFMAs per tile and group instead
// of 12 and two thirds of the activation bytes; the high terms and the low terms
// (times 2^11) accumulate apart and meet as hi + 2^-11 lo before the scale FMA,
// and the stored outputs are scaled back by 2^-E of their row (exact).
template <int F, int TM, int NS, int PF, bool F8, bool H2 = false>
__global__ __launch_bounds__(kW8Threads) void bf3_gemm_kernel(GemmArgs a) {
  static_assert(!F8 || F == F_W4A16, "the t16f8 layout holds int4 weights");
  static_assert(!H2 || F == F_W4A16, "two float16 terms: integer weights only");
  constexpr int T3 = H2 ? 2 : 3;  // activation terms per slot
  __shared__ __align__(16) float red[NS * TM * kW8Waves * kWave * 4];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int c = lane & 15;
  const int M = a.M, N = a.N, Kp = a.Kp, G = (Kp + 127) / 128, G4 = t16_groups(Kp);
  const int mb0 = blockIdx.y * TM, m0 = mb0 * 16;
  const int S = (N + 15) / 16;
  const int sbase = (int)((unsigned)S / gridDim.x), srem = S - sbase * (int)gridDim.x;
  const int bx = blockIdx.x;
  const int sb = bx * sbase + min(bx, srem), se = sb + sbase + (bx < srem ? 1 : 0);
  // K split over gridDim.z workgroups of a column: this one sums groups [g0, g1) and
  // writes its partial tile to its slice of a.ypart (gridDim.z == 1: all groups, Y)
  const int KS = gridDim.z, ks = blockIdx.z;
  const int gsl = (G + KS - 1) / KS;
  const int g0 = min(G, ks * gsl), g1 = min(G, g0 + gsl), GL = g1 - g0;
  const int nph = (GL + kW8Waves - 1) / kW8Waves;
  float *const yo = KS > 1 ? a.ypart + (size_t)ks * M * N : a.y;

  const Rsrc rx = make_rsrc(a.x3, (uint32_t)min(H2 ? x2h_bytes(M, Kp) : x3_bytes(M, Kp), (size_t)0xFFFFFFF0u));
  const Rsrc rw = make_rsrc(a.qw, (uint32_t)min(F8 ? t16f8_qw_bytes(N, Kp) : t16_qw_bytes(N, Kp),
                                                (size_t)0xFFFFFFF0u));
  const size_t gents = t16_group_entries(N, Kp);
  const Rsrc rs = make_rsrc(F == F_W4A16 ? (const void *)a.scales : (const void *)a.e8m0,
                            F == F_W4A16 ? (uint32_t)(gents * 4) : (uint32_t)t16_e8m0_bytes(N, Kp));
  const Rsrc rz = make_rsrc(a.zeros ? a.zeros : a.qw, (F == F_W4A16 && !F8 && a.zeros) ? (uint32_t)gents : 0u);
  const int zadd = (F == F_W4A16 && !a.zeros) ? 8 : 0;

  v4u xa[4][T3][TM];
  for (int cb = sb; cb < se; cb += NS) {
    const int ce = min(cb + NS, se);
    if (wave >= GL) {
      // no group in any phase (fewer than eight groups): this wave's partial tiles are zero
      for (int j = 0; j < ce - cb; j++)
#pragma unroll
        for (int i = 0; i < TM; i++)
          *reinterpret_cast<v4f *>(&red[(((j * TM + i) * kW8Waves + wave) * kWave + lane) * 4]) =
              v4f{0.f, 0.f, 0.f, 0.f};
    }
    for (int ph = 0; ph < nph; ph++) {
      const int g = g0 + ph * kW8Waves + wave;
      if (g >= g1) continue;  // wave-uniform: this wave has no group in the last phase
      // Each stage's address is one lane offset (shared by all stages) plus a
      // workgroup-uniform scalar offset: per-stage vector addresses would be
      // allocated to the registers of earlier stages' pending loads, which makes
      // every stage wait for the previous one. Stages past the chunk reload its
      // last subtile (in bounds; they fill LDS slots the reduction never reads).
      auto load = [&](B3Stage &st, int j) {
        const uint32_t sj = (uint32_t)min(cb + j, ce - 1);
        if constexpr (F8) {
          // the tile's two 1 KiB halves: lane bytes 0-15, then 16-31
          const uint32_t tb = (sj * G4 + g) * (2 * kWave * 16u);
          st.w = ld_b128(rw, (uint32_t)lane * 16u, tb);
          st.w2 = ld_b128(rw, (uint32_t)lane * 16u, tb + kWave * 16u);
        } else {
          st.w = ld_b128(rw, (uint32_t)lane * 16u, (sj * G4 + g) * (kWave * 16u));
        }
        if constexpr (F == F_W4A16) {
          // entry ((sj G4/4 + g/4) 16 + c) 4 + g % 4 of the group data
          const uint32_t gu = (sj * (G4 / 4) + g / 4) * 64u;
          st.s = ld_f32(rs, (uint32_t)c * 16u, (gu + (g & 3)) * 4u);
          if constexpr (!F8) st.z = ld_u32(rz, (uint32_t)c * 4u, gu);  // symmetric: a zero-length range reads 0
        } else {
          st.s = 0.0f;
          st.z = ld_u32(rs, (uint32_t)(lane & ~3), (sj * G4 + g) * kWave);
        }
      };
      // issue order = retirement order: the first subtile's weights, then the
      // activations, then the other PF subtiles of the chunk (all unconditional:
      // stages past the chunk read zero-length ranges, and a later chunk reloads
      // the activations from the cache, so the waits are exact)
      B3Stage st[PF + 1];
      load(st[0], 0);
      {
#pragma unroll
        for (int u = 0; u < 4; u++)
#pragma unroll
          for (int p = 0; p < T3; p++)
#pragma unroll
            for (int i = 0; i < TM; i++) {
              // row blocks past the last one read zeros (past the descriptor)
              const uint32_t off = ((((uint32_t)(mb0 + i) * G + g) * 4 + u) * T3 + p) * kWave * 16 + lane * 16;
              const uint4 v = ld_b128(rx, off);
              xa[u][p][i] = v4u{v.x, v.y, v.z, v.w};
            }
      }
      // the scheduler would otherwise group the loads by type, moving each
      // subtile's scales behind every later weight load
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 1; j <= PF; j++) {
        load(st[j], j);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int j = 0; j < NS; j++) {
        // only the last slot is guarded (workgroups get floor or ceil of the
        // average share): earlier subtiles past the chunk (a short last chunk)
        // read zero-length ranges and fill LDS slots the reduction never reads,
        // so most of the unrolled loop is one basic block and the scheduler can
        // decode the next subtile under this one's MFMAs
        if (j == NS - 1 && cb + j >= ce) continue;
        B3Stage &cur = st[j % (PF + 1)];
        v4f *slot = reinterpret_cast<v4f *>(&red[((j * TM * kW8Waves + wave) * kWave + lane) * 4]);
        v4f prev[TM];  // the earlier phases' sum of this subtile (read ahead of the MFMAs)
#pragma unroll
        for (int i = 0; i < TM; i++) {
          const v4f t = slot[i * kW8Waves * kWave];  // unconditional: a select, not a branch
          prev[i] = ph == 0 ? v4f{0.f, 0.f, 0.f, 0.f} : t;
        }
        v4u b[4];
        float fs;
        if constexpr (F8) {
          // operand u, element e = lane byte 8u + e
          const uint32_t wd[8] = {cur.w.x, cur.w.y, cur.w.z, cur.w.w, cur.w2.x, cur.w2.y, cur.w2.z, cur.w2.w};
#pragma unroll
          for (int u = 0; u < 4; u++) {
            if constexpr (H2) {
              b[u][0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(wd[2 * u], 512.0f, false));
              b[u][1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(wd[2 * u], 512.0f, true));
              b[u][2] =
                  __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(wd[2 * u + 1], 512.0f, false));
              b[u][3] =
                  __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(wd[2 * u + 1], 512.0f, true));
            } else {
              b[u][0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wd[2 * u], 512.0f, false));
              b[u][1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wd[2 * u], 512.0f, true));
              b[u][2] =
                  __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wd[2 * u + 1], 512.0f, false));
              b[u][3] =
                  __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wd[2 * u + 1], 512.0f, true));
            }
          }
          fs = cur.s;
        } else if constexpr (F == F_W4A16) {
          const float zf = (float)(int)(((cur.z >> (8 * (g & 3))) & 0xFFu) + (uint32_t)zadd);
          const uint32_t wd[4] = {cur.w.x, cur.w.y, cur.w.z, cur.w.w};
#pragma unroll
          for (int h = 0; h < 2; h++)  // u = h: low nibbles of bytes 8h .. 8h+7; u = 2 + h: high nibbles
#pragma unroll
            for (int d = 0; d < 2; d++) {
              uint32_t x0, x1;
              if constexpr (H2) w4_f16x4(lo_nibbles(wd[2 * h + d]), zf, x0, x1);
              else w4_bf16x4(lo_nibbles(wd[2 * h + d]), zf, x0, x1);
              b[h][2 * d] = x0;
              b[h][2 * d + 1] = x1;
              if constexpr (H2) w4_f16x4(hi_nibbles(wd[2 * h + d]), zf, x0, x1);
              else w4_bf16x4(hi_nibbles(wd[2 * h + d]), zf, x0, x1);
              b[2 + h][2 * d] = x0;
              b[2 + h][2 * d + 1] = x1;
            }
          fs = cur.s;
        } else {
          // the MFMA sums the four blocks of group g of row c (lanes c, c+16, c+32,
          // c+48): each block's codes carry 2^(e - emax), exact in bf16 down to
          // 2^-126; the fp32 factor 2^(emax - 127) (NaN for 255) follows the MFMA
          const int e = (int)((cur.z >> (8 * (lane & 3))) & 0xFFu);
          int emax = max(e, __shfl_xor(e, 16));
          emax = max(emax, __shfl_xor(emax, 32));
          const int dexp = e - emax;
          const float bs = dexp >= -126 ? __uint_as_float((uint32_t)(dexp + 127) << 23) : 0.0f;
          const uint32_t wd[4] = {cur.w.x, cur.w.y, cur.w.z, cur.w.w};
#pragma unroll
          for (int u = 0; u < 4; u++) {
            b[u][0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd[u], bs, 0));
            b[u][1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd[u], bs, 1));
            b[u][2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd[u], bs, 2));
            b[u][3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd[u], bs, 3));
          }
          fs = e8m0_to_f32((uint32_t)emax);
        }
#pragma unroll
        for (int i = 0; i < TM; i++) {
          v4f dacc = {0.f, 0.f, 0.f, 0.f};
          if constexpr (H2) {
            v4f dlo = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < 4; u++) {
              dacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, xa[u][0][i]),
                                                            __builtin_bit_cast(v8h, b[u]), dacc, 0, 0, 0);
              dlo = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, xa[u][T3 - 1][i]),
                                                           __builtin_bit_cast(v8h, b[u]), dlo, 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < 4; r++) dacc[r] = __builtin_fmaf(dlo[r], 0x1p-11f, dacc[r]);
          } else {
#pragma unroll
            for (int u = 0; u < 4; u++)
#pragma unroll
              for (int p = 0; p < T3; p++)
                dacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, xa[u][p][i]),
                                                               __builtin_bit_cast(v8bf, b[u]), dacc, 0, 0, 0);
          }
          v4f f;
#pragma unroll
          for (int r = 0; r < 4; r++) f[r] = __builtin_fmaf(fs, dacc[r], prev[i][r]);
          slot[i * kW8Waves * kWave] = f;
        }
        if (j + PF + 1 < NS) load(cur, j + PF + 1);
      }
    }
    // ---- reduce the waves' partial tiles of the chunk and store
    __syncthreads();
    for (int e = threadIdx.x; e < (ce - cb) * TM * kWave; e += kW8Threads) {
      const int l = e % kWave, i = (e / kWave) % TM, j = e / (kWave * TM);
      v4f v = *reinterpret_cast<const v4f *>(&red[(((j * TM + i) * kW8Waves + 0) * kWave + l) * 4]);
#pragma unroll
      for (int w = 1; w < kW8Waves; w++) {
        const v4f t = *reinterpret_cast<const v4f *>(&red[(((j * TM + i) * kW8Waves + w) * kWave + l) * 4]);
        v += t;
      }
      const int n = 16 * (cb + j) + (l & 15), lr = 16 * i + 4 * (l >> 4);
      if (n < N) {
#pragma unroll
        for (int r = 0; r < 4; r++)
          if (m0 + lr + r < M) yo[(size_t)(m0 + lr + r) * N + n] = H2 ? ldexpf(v[r], -a.xexp[m0 + lr + r]) : v[r];
      }
    }
    __syncthreads();  // red is rewritten by the next chunk
  }
}

// y = the K slices' partial outputs added in slice order (deterministic).
__global__ __launch_bounds__(256) void bf3_reduce_kernel(const float *__restrict__ part, int ks, size_t n,
                                                         float *__restrict__ y) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  float t = part[i];
  for (int k = 1; k < ks; k++) t += part[(size_t)k * n + i];
  y[i] = t;
}

// Largest chunk (its partial tiles fill NS * TM * 8 KiB of LDS) and weight subtiles
// in flight (PF + 1 stages of 6 registers) that compile without spills.
template <int TM> struct B3Cfg {
  static constexpr int NS = TM >= 2 ? 6 : 12;
  static constexpr int PF = NS - 1;
};

// Grid of the bf16x3 GEMM: gy row blocks of 16 TM rows, gx workgroups over the
// S = ceil(N/16) subtiles, spw subtiles for the busiest workgroup.
static void bf3_grid(int M, int N, int TM, int cus, int &gx, int &gy, int &spw) {
  const int S = (N + 15) / 16;
  gy = (M + 16 * TM - 1) / (16 * TM);
  gx = std::max(1, std::min(S, cus / gy));
  spw = (S + gx - 1) / gx;
}

template <int F, int TM, bool F8, bool H2 = false>
static void launch_bf3_t(const GemmArgs &a, int cus, int ks, hipStream_t s) {
  constexpr int NS = B3Cfg<TM>::NS, PF = B3Cfg<TM>::PF;
  // every subtile slot of a chunk but the last is computed, so the chunk length
  // is the workgroup's share (up to NS; its loads all in flight)
  int gx, gy, spw;
  bf3_grid(a.M, a.N, TM, cus, gx, gy, spw);
  if (ks > 1) {
    // a K split keeps one workgroup per CU: ks times fewer columns, each CU with
    // ks times the subtiles over 1/ks of K (and of the activation terms)
    gx = std::max(1, gx / ks);
    spw = ((a.N + 15) / 16 + gx - 1) / gx;
  }
  auto go = [&](auto ns) {
    constexpr int C = decltype(ns)::value < NS ? decltype(ns)::value : NS;
    hipLaunchKernelGGL((bf3_gemm_kernel<F, TM, C, (C - 1 < PF ? C - 1 : PF), F8, H2>), dim3(gx, gy, ks),
                       dim3(kW8Threads), 0, s, a);
  };
  switch (spw) {
    case 1: go(std::integral_constant<int, 1>{}); break;
    case 2: go(std::integral_constant<int, 2>{}); break;
    case 3: go(std::integral_constant<int, 3>{}); break;
    case 4: go(std::integral_constant<int, 4>{}); break;
    case 5: go(std::integral_constant<int, 5>{}); break;
    case 6: go(std::integral_constant<int, 6>{}); break;
    case 7:
    case 8: go(std::integral_constant<int, 8>{}); break;
    default: go(std::integral_constant<int, NS>{}); break;
  }
}

bool w4a16_prefers_t16f8(int M, int N, int Kp, int num_cus) {
  // Subtiles per workgroup of the launch as it runs (after a K split). Measured at 64 x
  // 11008 x 4096 (6 subtiles per workgroup), 128 x 11008 x 4096 (11), 256 x 4096 x 4096
  // (8) and 512 x 4096 x 4096 (16), t16f8 took 3-11 % less time with the weights cold
  // and 5-15 % less hot; with 2 or 3 subtiles per workgroup (16 and 32 x 11008 x 4096,
  // and at K = 11008 16 and 32 rows split in two) its twice as many weight bytes per
  // stage cost more than the conversions it saves when cold (5-13 % more time). At 64
  // x 4096 x 11008 split in two (4 subtiles) t16f8 took 27.2 against 30.2 us hot, 32.1
  // against 32.3 cold; 128 x 4096 x 11008 unsplit (4), 43.3 against 49.6 hot.
  int gx, gy, spw;
  const int cus = num_cus > 0 ? num_cus : 256;
  bf3_grid(M, N, M > 16 ? 2 : 1, cus, gx, gy, spw);
  const int ks = bf3_k_slices(F_W4A16, M, Kp);
  if (ks > 1) spw = ((N + 15) / 16 + std::max(1, gx / ks) - 1) / std::max(1, gx / ks);
  return spw >= 4;
}

// K slices: each CU reads its rows' activation terms (6 bytes per element) for all
// of K, ~1 MB at 16 x 11008, which bounds these shapes; a split reads 1/ks of them
// per CU at the cost of a reduce launch (~1.6 us in a graph) and ks times the
// subtiles per workgroup. Measured (hot): 16 x 4096 x 11008 W4A16 18.5 -> 16.4 us
// (2), MXFP4 17.2 -> 14.2 us (4); 64 x 4096 x 11008 W4A16 36.7 -> 32.9 us (2), MXFP4
// 29.2 -> 28.9 (2, not taken); at K = 4096 every split lost (13.8 -> 15.7 us at 16 x
// 11008 x 4096), and with two row blocks more subtiles mean more chunks, each
// reloading the activations. W4A16 above 64 rows is not split: at 128 x 4096 x 11008
// the split took 65.9 against 49.6 us hot on t16 (57.8 against 43.3 on t16f8); 256
// rows gained 8 % (94.8 against 102.8 on t16f8), too little for a partial-output
// workspace that grows with M (ks M N 4 bytes, 256 MiB at 8192 x 4096 x 11008).
// Since W4A16 reads two float16 terms (4 bytes per element) one row block no longer
// gains from the split (hot, split against unsplit: 16 x 4096 x 11008 16.3-16.5
// against 15.4 us, 16 x 11008 x 11008 28.2 against 26.9, 16 x 4096 x 8192 13.7-14.0
// against 12.9) while two or more still do (32 x 4096 x 11008 21.1-21.2 against
// 25.0, 64 x 4096 x 11008 26.0-26.3 against 27.6-27.8; 64 x 4096 x 8192 even).
int bf3_k_slices(int fmt, int M, int Kp) {
  if (Kp < 8192) return 1;
  if (fmt == F_MXFP4) return M <= 16 ? 4 : 1;
  return fmt == F_W4A16 && M > 16 && M <= 64 ? 2 : 1;
}

size_t bf3_part_bytes(int fmt, int M, int N, int Kp) {
  const int ks = bf3_k_slices(fmt, M, Kp);
  return ks > 1 ? (size_t)ks * M * N * sizeof(float) : 0;
}

hipError_t launch_bf3_gemm(int fmt, const GemmArgs &a, int num_cus, hipStream_t s, bool f8) {
  const int cus = num_cus > 0 ? num_cus : 256;
  if (!a.x3 || !a.wt16 || (f8 && fmt != F_W4A16)) return hipErrorInvalidValue;
  // the split only where the caller gave room for its partial outputs
  const int ks = a.ypart ? bf3_k_slices(fmt, a.M, a.Kp) : 1;
  // W4A16: 32-row blocks halve the weight decode per output once there are two
  // row blocks (its decode VALU, not bytes, bounds it). MXFP4 decodes with a few
  // conversion instructions, and each CU's bytes matter more: the activation terms
  // (6 B per element of its 16 TM rows) plus its share of the weights, the
  // smaller of TM = 1 and 2 once it saves a quarter (16-row blocks, which decode
  // each weight twice as often, win at N = 4096 and K = 11008, saving ~38 %, and
  // lose slightly at M = 64 x 11008 x 4096, saving 21 %).
  bool tall = a.M > 16;
  if (fmt == F_MXFP4 && tall) {
    auto cu_bytes = [&](int tm) {
      const int gy = (a.M + 16 * tm - 1) / (16 * tm), S = (a.N + 15) / 16;
      const int gx = std::max(1, std::min(S, cus / gy));
      const double spw = (double)((S + gx - 1) / gx);
      return (double)tm * 16 * a.Kp * 6 + spw * 16 * (a.Kp / 2 + a.Kp / 32);
    };
    tall = cu_bytes(1) > 0.75 * cu_bytes(2);
  }
  if (fmt == F_W4A16 && !a.xexp) return hipErrorInvalidValue;  // W4A16 reads the two-term split
  if (fmt == F_W4A16 && f8) {
    if (tall) launch_bf3_t<F_W4A16, 2, true, true>(a, cus, ks, s);
    else launch_bf3_t<F_W4A16, 1, true, true>(a, cus, ks, s);
  } else if (fmt == F_W4A16) {
    if (tall) launch_bf3_t<F_W4A16, 2, false, true>(a, cus, ks, s);
    else launch_bf3_t<F_W4A16, 1, false, true>(a, cus, ks, s);
  } else if (fmt == F_MXFP4) {
    if (tall) launch_bf3_t<F_MXFP4, 2, false>(a, cus, ks, s);
    else launch_bf3_t<F_MXFP4, 1, false>(a, cus, ks, s);
  } else {
    return hipErrorInvalidValue;
  }
  if (ks > 1) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const size_t n = (size_t)a.M * a.N;
    hipLaunchKernelGGL(bf3_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a.ypart, ks, n, a.y);
  }
  return hipGetLastError();
}

// ============================================================ W4A16 / MXFP4, fp32 MFMA
//
// K is walked in chunks of 128 elements (one int4 group, or four MXFP4 blocks);
// waves split the chunks. Lane (q, c) loads the 16 bytes at row offset
// 64*chunk + 16q, i.e.
//   int4 : group `chunk`, low nibbles at k = 128*chunk + 16q + u, high at +64
//   MXFP4: block 4*chunk + q, low nibbles at k = 128*chunk + 32q + u, high at +16
// (u = byte 0..15). Byte u feeds two MFMA k-slots: (low, high). The int4 group
// product is accumulated unscaled ((q - z) is exact in fp32) and rescaled by s
// once per group; MXFP4 weights carry their power-of-two block scale exactly.
template <int F, int TM, int TN>
__global__ __launch_bounds__(kThreads) void f32_mfma_kernel(GemmArgs a) {
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int q = lane >> 4, c = lane & 15;
  const int M = a.M, N = a.N, Kp = a.Kp;
  const size_t rowbytes = (size_t)(Kp >> 1);
  const int nchunk = (Kp + 127) >> 7;
  const int G = Kp / kGroup, B = Kp / kMxBlock;
  const int n0 = blockIdx.x * 16 * TN, m0 = blockIdx.y * 16 * TM;
  constexpr int kHiOff = (F == F_MXFP4) ? 16 : 64;

  int nrow[TN], mrow[TM];
  bool nok[TN], mok[TM];
#pragma unroll
  for (int j = 0; j < TN; j++) {
    const int n = n0 + 16 * j + c;
    nok[j] = n < N;
    nrow[j] = nok[j] ? n : N - 1;
  }
#pragma unroll
  for (int i = 0; i < TM; i++) {
    const int m = m0 + 16 * i + c;
    mok[i] = m < M;
    mrow[i] = mok[i] ? m : M - 1;
  }
  v4f facc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) facc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  for (int ch = wave; ch < nchunk; ch += kWaves) {
    const bool kok = (F == F_MXFP4) ? (4 * ch + q < B) : true;
    const int kbase = (F == F_MXFP4) ? 128 * ch + 32 * q : 128 * ch + 16 * q;
    uint4 w[TN];
    float zf[TN], sc[TN];
#pragma unroll
    for (int j = 0; j < TN; j++) {
      w[j] = kok ? *reinterpret_cast<const uint4 *>(a.qw + nrow[j] * rowbytes + (size_t)ch * 64 + q * 16)
                 : make_uint4(0, 0, 0, 0);
      if constexpr (F == F_MXFP4) {
        sc[j] = (kok && nok[j]) ? e8m0_to_f32(a.e8m0[(size_t)nrow[j] * B + 4 * ch + q]) : 0.0f;
      } else {
        sc[j] = a.scales[(size_t)nrow[j] * G + ch];
        zf[j] = a.zeros ? (float)a.zeros[(size_t)nrow[j] * G + ch] : 8.0f;
        if (!nok[j]) zf[j] = 0.0f, w[j] = make_uint4(0, 0, 0, 0);
      }
    }
    v4f dacc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < TN; j++) dacc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

#pragma unroll
    for (int d = 0; d < 4; d++) {
      float4 xlo[TM], xhi[TM];
#pragma unroll
      for (int i = 0; i < TM; i++) {
        const float *xr = a.x + (size_t)mrow[i] * Kp + kbase + 4 * d;
        if (mok[i] && kok) {
          xlo[i] = *reinterpret_cast<const float4 *>(xr);
          xhi[i] = *reinterpret_cast<const float4 *>(xr + kHiOff);
        } else {
          xlo[i] = make_float4(0.f, 0.f, 0.f, 0.f);
          xhi[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
      float wl[TN][4], wh[TN][4];
#pragma unroll
      for (int j = 0; j < TN; j++) {
        const uint32_t wd = d == 0 ? w[j].x : d == 1 ? w[j].y : d == 2 ? w[j].z : w[j].w;
        if constexpr (F == F_MXFP4) {
          const v2f p0 = e2m1_pair<0>(wd, sc[j]), p1 = e2m1_pair<1>(wd, sc[j]);
          const v2f p2 = e2m1_pair<2>(wd, sc[j]), p3 = e2m1_pair<3>(wd, sc[j]);
          wl[j][0] = p0.x; wh[j][0] = p0.y; wl[j][1] = p1.x; wh[j][1] = p1.y;
          wl[j][2] = p2.x; wh[j][2] = p2.y; wl[j][3] = p3.x; wh[j][3] = p3.y;
        } else {
          const uint32_t lo = lo_nibbles(wd), hi = hi_nibbles(wd);
#pragma unroll
          for (int u = 0; u < 4; u++) {
            wl[j][u] = (float)((lo >> (8 * u)) & 0xFF) - zf[j];
            wh[j][u] = (float)((hi >> (8 * u)) & 0xFF) - zf[j];
          }
        }
      }
#pragma unroll
      for (int u = 0; u < 4; u++) {
#pragma unroll
        for (int i = 0; i < TM; i++) {
          const float xa = u == 0 ? xlo[i].x : u == 1 ? xlo[i].y : u == 2 ? xlo[i].z : xlo[i].w;
          const float xb = u == 0 ? xhi[i].x : u == 1 ? xhi[i].y : u == 2 ? xhi[i].z : xhi[i].w;
#pragma unroll
          for (int j = 0; j < TN; j++) {
            if constexpr (F == F_MXFP4) {
              facc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa, wl[j][u], facc[i][j], 0, 0, 0);
              facc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(xb, wh[j][u], facc[i][j], 0, 0, 0);
            } else {
              dacc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa, wl[j][u], dacc[i][j], 0, 0, 0);
              dacc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(xb, wh[j][u], dacc[i][j], 0, 0, 0);
            }
          }
        }
      }
    }
    if constexpr (F == F_W4A16) {
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
          for (int r = 0; r < 4; r++) facc[i][j][r] = __builtin_fmaf(sc[j], dacc[i][j][r], facc[i][j][r]);
    }
  }
  constexpr int NV = TM * TN * 4;
  __shared__ float red[kWaves][NV][kWave];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) red[wave][(i * TN + j) * 4 + r][lane] = facc[i][j][r];
  __syncthreads();
  for (int idx = wave; idx < NV; idx += kWaves) {
    const int i = idx / (TN * 4), j = (idx / 4) % TN, r = idx % 4;
    const float t = (red[0][idx][lane] + red[1][idx][lane]) + (red[2][idx][lane] + red[3][idx][lane]);
    const int m = m0 + 16 * i + 4 * q + r, n = n0 + 16 * j + c;
    if (m < M && n < N) a.y[(size_t)m * N + n] = t;
  }
}

template <int F, int TM>
static hipError_t launch_f32_tm(const GemmArgs &a, hipStream_t s) {
  constexpr int TN = 2;
  dim3 grid((a.N + 16 * TN - 1) / (16 * TN), (a.M + 16 * TM - 1) / (16 * TM));
  hipLaunchKernelGGL((f32_mfma_kernel<F, TM, TN>), grid, dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_f32_mfma(int fmt, const GemmArgs &a, hipStream_t s) {
  if (fmt == F_W4A16) {
    if (a.M <= 16) return launch_f32_tm<F_W4A16, 1>(a, s);
    if (a.M <= 32) return launch_f32_tm<F_W4A16, 2>(a, s);
    return launch_f32_tm<F_W4A16, 4>(a, s);
  }
  if (fmt == F_MXFP4) {
    if (a.M <= 16) return launch_f32_tm<F_MXFP4, 1>(a, s);
    if (a.M <= 32) return launch_f32_tm<F_MXFP4, 2>(a, s);
    return launch_f32_tm<F_MXFP4, 4>(a, s);
  }
  return hipErrorInvalidValue;
}

// ============================================================ group accumulators (dot4 path)
//
// out[m, n, g] through exactly the integer arithmetic the W4A8 GEMV uses: for
// each 16-byte chunk of the group, eight dot4 of unsigned codes and int8
// activations, then minus z * asum.
__global__ __launch_bounds__(kThreads) void groupacc_dot4_kernel(
    const int8_t *__restrict__ xq, const int32_t *__restrict__ asum, int M, int Kp,
    const uint8_t *__restrict__ qw, const uint8_t *__restrict__ zeros, int N,
    int32_t *__restrict__ out) {
  const int G = Kp / kGroup;
  const size_t total = (size_t)M * N * G;
  for (size_t t = (size_t)blockIdx.x * kThreads + threadIdx.x; t < total; t += (size_t)gridDim.x * kThreads) {
    const int g = (int)(t % G);
    const int n = (int)((t / G) % N);
    const int m = (int)(t / ((size_t)G * N));
    const uint8_t *wrow = qw + (size_t)n * (Kp >> 1) + (size_t)g * 64;
    const int8_t *arow = xq + (size_t)m * Kp + (size_t)g * kGroup;
    int d = 0;
#pragma unroll
    for (int b = 0; b < 4; b++) {
      const uint4 w = *reinterpret_cast<const uint4 *>(wrow + 16 * b);
      const uint4 al = *reinterpret_cast<const uint4 *>(arow + 16 * b);
      const uint4 ah = *reinterpret_cast<const uint4 *>(arow + 64 + 16 * b);
      d = __builtin_amdgcn_sdot4((int)lo_nibbles(w.x), (int)al.x, d, false);
      d = __builtin_amdgcn_sdot4((int)hi_nibbles(w.x), (int)ah.x, d, false);
      d = __builtin_amdgcn_sdot4((int)lo_nibbles(w.y), (int)al.y, d, false);
      d = __builtin_amdgcn_sdot4((int)hi_nibbles(w.y), (int)ah.y, d, false);
      d = __builtin_amdgcn_sdot4((int)lo_nibbles(w.z), (int)al.z, d, false);
      d = __builtin_amdgcn_sdot4((int)hi_nibbles(w.z), (int)ah.z, d, false);
      d = __builtin_amdgcn_sdot4((int)lo_nibbles(w.w), (int)al.w, d, false);
      d = __builtin_amdgcn_sdot4((int)hi_nibbles(w.w), (int)ah.w, d, false);
    }
    const int z = zeros ? (int)zeros[(size_t)n * G + g] : 8;
    out[t] = d - z * asum[(size_t)m * G + g];
  }
}

hipError_t launch_groupacc_dot4(const int8_t *xq, const int32_t *asum, int M, int Kp,
                                const uint8_t *qw, const uint8_t *zeros, int N,
                                int32_t *out, hipStream_t s) {
  const size_t total = (size_t)M * N * (Kp / kGroup);
  size_t blocks = (total + kThreads - 1) / kThreads;
  if (blocks > 65536) blocks = 65536;
  if (blocks == 0) blocks = 1;
  hipLaunchKernelGGL(groupacc_dot4_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, s, xq, asum, M, Kp, qw,
                     zeros, N, out);
  return hipGetLastError();
}

// ============================================================ t16 repack
//
// One thread per 16-byte lane chunk of qwt (reads the 16 bytes of the row-major
// matrix it holds, or writes zeros for padding), then one per group entry of
// st / zt. A one-time layout change of resident weights, not a timed path.
__global__ __launch_bounds__(kThreads) void repack_int4_t16_kernel(const uint8_t *__restrict__ qw,
                                                                    const float *__restrict__ scales,
                                                                    const uint8_t *__restrict__ zeros, int N, int Kp,
                                                                    uint8_t *__restrict__ qwt, float *__restrict__ st,
                                                                    uint8_t *__restrict__ zt) {
  const int G = Kp / kGroup, G4 = t16_groups(Kp);
  const size_t rowbytes = (size_t)(Kp >> 1);
  const size_t nchunk = t16_qw_bytes(N, Kp) / 16, nent = t16_group_entries(N, Kp);
  const size_t stride = (size_t)gridDim.x * kThreads;
  for (size_t t = (size_t)blockIdx.x * kThreads + threadIdx.x; t < nchunk; t += stride) {
    const int l = (int)(t % 64), g = (int)((t / 64) % G4);
    const size_t sub = t / (64 * (size_t)G4);
    const size_t row = sub * 16 + (l & 15);
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (row < (size_t)N && g < G)
      v = *reinterpret_cast<const uint4 *>(qw + row * rowbytes + (size_t)g * 64 + (size_t)(l >> 4) * 16);
    reinterpret_cast<uint4 *>(qwt)[t] = v;
  }
  for (size_t e = (size_t)blockIdx.x * kThreads + threadIdx.x; e < nent; e += stride) {
    // e = ((s * G4/4 + g/4) * 16 + c) * 4 + g % 4
    const int j = (int)(e % 4), c = (int)((e / 4) % 16);
    const size_t gq = (e / 64) % (size_t)(G4 / 4), sub = e / (64 * (size_t)(G4 / 4));
    const size_t row = sub * 16 + c;
    const int g = (int)(gq * 4) + j;
    const bool ok = row < (size_t)N && g < G;
    st[e] = ok ? scales[row * G + g] : 0.0f;
    if (zt) zt[e] = (ok && zeros) ? zeros[row * G + g] : (uint8_t)0;
  }
}

// t16f8: one thread per 16-byte chunk of qwt8 (half h of lane l of tile (s, g)):
// nibble h of the 16 source bytes the t16 lane holds, less the group's zero-point,
// as E4M3 sign-magnitude bytes; then the scales as for t16.
__device__ __forceinline__ uint32_t e4m3_small_int(int d) {
  const int n = d < 0 ? -d : d;
  if (n > 15) return 0x7Fu;  // not exact in this encoding: NaN
  return (d < 0 ? 0x80u : 0u) | (uint32_t)n;  // n 2^-9: subnormal below 8, exponent field 1 from 8
}

__global__ __launch_bounds__(kThreads) void repack_int4_t16f8_kernel(const uint8_t *__restrict__ qw,
                                                                      const float *__restrict__ scales,
                                                                      const uint8_t *__restrict__ zeros, int N,
                                                                      int Kp, uint8_t *__restrict__ qwt8,
                                                                      float *__restrict__ st) {
  const int G = Kp / kGroup, G4 = t16_groups(Kp);
  const size_t rowbytes = (size_t)(Kp >> 1);
  const size_t nchunk = t16f8_qw_bytes(N, Kp) / 16, nent = t16_group_entries(N, Kp);
  const size_t stride = (size_t)gridDim.x * kThreads;
  for (size_t t = (size_t)blockIdx.x * kThreads + threadIdx.x; t < nchunk; t += stride) {
    const int l = (int)(t % 64), h = (int)((t / 64) % 2), g = (int)((t / 128) % G4);
    const size_t sub = t / (128 * (size_t)G4);
    const size_t row = sub * 16 + (l & 15);
    uint32_t o[4] = {0u, 0u, 0u, 0u};
    if (row < (size_t)N && g < G) {
      const uint4 v = *reinterpret_cast<const uint4 *>(qw + row * rowbytes + (size_t)g * 64 + (size_t)(l >> 4) * 16);
      const int z = zeros ? (int)zeros[row * G + g] : 8;
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int d = 0; d < 4; d++)
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const int code = (int)((w[d] >> (8 * k + 4 * h)) & 0xFu);
          o[d] |= e4m3_small_int(code - z) << (8 * k);
        }
    }
    reinterpret_cast<uint4 *>(qwt8)[t] = make_uint4(o[0], o[1], o[2], o[3]);
  }
  for (size_t e = (size_t)blockIdx.x * kThreads + threadIdx.x; e < nent; e += stride) {
    const int j = (int)(e % 4), c = (int)((e / 4) % 16);
    const size_t gq = (e / 64) % (size_t)(G4 / 4), sub = e / (64 * (size_t)(G4 / 4));
    const size_t row = sub * 16 + c;
    const int g = (int)(gq * 4) + j;
    st[e] = (row < (size_t)N && g < G) ? scales[row * G + g] : 0.0f;
  }
}

// MXFP4: the same qwt order over rows of Kp/2 bytes (a multiple of 16; chunks past
// the row are zero), then the E8M0 byte of each lane's block in lane order.
__global__ __launch_bounds__(kThreads) void repack_mxfp4_t16_kernel(const uint8_t *__restrict__ qw,
                                                                     const uint8_t *__restrict__ e8m0, int N, int Kp,
                                                                     uint8_t *__restrict__ qwt,
                                                                     uint8_t *__restrict__ et) {
  const int G4 = t16_groups(Kp), B = Kp / kMxBlock;
  const size_t rowbytes = (size_t)(Kp >> 1);
  const size_t nchunk = t16_qw_bytes(N, Kp) / 16;  // = entries of et
  const size_t stride = (size_t)gridDim.x * kThreads;
  for (size_t t = (size_t)blockIdx.x * kThreads + threadIdx.x; t < nchunk; t += stride) {
    const int l = (int)(t % 64), g = (int)((t / 64) % G4);
    const size_t sub = t / (64 * (size_t)G4);
    const size_t row = sub * 16 + (l & 15);
    const int blk = 4 * g + (l >> 4);
    const bool ok = row < (size_t)N && blk < B;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (ok) v = *reinterpret_cast<const uint4 *>(qw + row * rowbytes + (size_t)blk * 16);
    reinterpret_cast<uint4 *>(qwt)[t] = v;
    et[t] = ok ? e8m0[row * B + blk] : (uint8_t)0;
  }
}

hipError_t launch_repack_mxfp4_t16(const uint8_t *qw, const uint8_t *e8m0, int N, int Kp, uint8_t *qwt, uint8_t *et,
                                   hipStream_t s) {
  const size_t work = t16_qw_bytes(N, Kp) / 16;
  size_t blocks = (work + kThreads - 1) / kThreads;
  if (blocks > 16384) blocks = 16384;
  if (blocks == 0) blocks = 1;
  hipLaunchKernelGGL(repack_mxfp4_t16_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, s, qw, e8m0, N, Kp, qwt, et);
  return hipGetLastError();
}

hipError_t launch_repack_int4_t16(const uint8_t *qw, const float *scales, const uint8_t *zeros, int N, int Kp,
                                  uint8_t *qwt, float *st, uint8_t *zt, hipStream_t s) {
  const size_t work = t16_qw_bytes(N, Kp) / 16;
  size_t blocks = (work + kThreads - 1) / kThreads;
  if (blocks > 16384) blocks = 16384;
  if (blocks == 0) blocks = 1;
  hipLaunchKernelGGL(repack_int4_t16_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, s, qw, scales, zeros, N, Kp,
                     qwt, st, zt);
  return hipGetLastError();
}

hipError_t launch_repack_int4_t16f8(const uint8_t *qw, const float *scales, const uint8_t *zeros, int N, int Kp,
                                    uint8_t *qwt8, float *st, hipStream_t s) {
  const size_t work = t16f8_qw_bytes(N, Kp) / 16;
  size_t blocks = (work + kThreads - 1) / kThreads;
  if (blocks > 16384) blocks = 16384;
  if (blocks == 0) blocks = 1;
  hipLaunchKernelGGL(repack_int4_t16f8_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, s, qw, scales, zeros, N,
                     Kp, qwt8, st);
  return hipGetLastError();
}

// ============================================================ copy (traffic calibration)

__global__ __launch_bounds__(kThreads) void copy16_kernel(uint4 *__restrict__ dst, const uint4 *__restrict__ src,
                                                          size_t n16) {
  for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n16; i += (size_t)gridDim.x * kThreads)
    dst[i] = src[i];
}

hipError_t launch_copy(void *dst, const void *src, size_t bytes, hipStream_t s) {
  const size_t n16 = bytes / 16;
  size_t blocks = (n16 + kThreads - 1) / kThreads;
  if (blocks > 8192) blocks = 8192;
  if (blocks == 0) blocks = 1;
  hipLaunchKernelGGL(copy16_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, s, static_cast<uint4 *>(dst),
                     static_cast<const uint4 *>(src), n16);
  return hipGetLastError();
}

}  // namespace lbk
