// Measurement kernels: a plain streaming read of a buffer, the reference point the
// decode GEMVs are measured against (the fastest a launch of that many bytes can
// read them), in the configurations the sweep in bench.py tries; VALU issue-rate
// probes of single instruction forms; an empty kernel (the fixed cost of a launch).
#include <hip/hip_runtime.h>

#include <utility>

#include "lb_device.h"
#include "lb_internal.h"

namespace lbk {

// Workgroup w reads the 16-byte units [w * per_wg, (w + 1) * per_wg) of the buffer,
// thread t the units t, t + T, ... of that range, U loads in flight per iteration
// (all issued before the first is used). Units past the buffer read 0 through the
// descriptor. The XOR of everything read is stored only if it equals a constant, so
// no load can be dropped and the kernel writes (almost surely) nothing; `sink` is
// one dword.
template <int T, int U>
__global__ __launch_bounds__(T) void stream_read_kernel(const uint8_t *src, uint32_t bytes, uint32_t per_wg,
                                                        uint32_t *sink) {
  const uint32_t first = blockIdx.x * per_wg;
  if (first * 16ull >= bytes) return;
  const uint32_t units = min(per_wg, (uint32_t)((bytes - first * 16ull) / 16));
  const Rsrc r = make_rsrc(src + (size_t)first * 16, units * 16);
  uint4 acc = make_uint4(0, 0, 0, 0);
  for (uint32_t base = 0; base < units; base += T * U) {
    uint4 v[U];
#pragma unroll
    for (int u = 0; u < U; u++) v[u] = ld_b128(r, (base + u * T + threadIdx.x) * 16);
#pragma unroll
    for (int u = 0; u < U; u++) {
      acc.x ^= v[u].x;
      acc.y ^= v[u].y;
      acc.z ^= v[u].z;
      acc.w ^= v[u].w;
    }
  }
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9E3779B9u) sink[0] = acc.x;
}

template <int T>
static hipError_t launch_read_t(const void *src, uint32_t bytes, int wgs, int loads, uint32_t *sink, hipStream_t s) {
  const uint32_t n16 = bytes / 16;
  const uint32_t per_wg = (n16 + wgs - 1) / wgs;
  const auto *p = static_cast<const uint8_t *>(src);
  switch (loads) {
    case 1: hipLaunchKernelGGL((stream_read_kernel<T, 1>), dim3(wgs), dim3(T), 0, s, p, bytes, per_wg, sink); break;
    case 2: hipLaunchKernelGGL((stream_read_kernel<T, 2>), dim3(wgs), dim3(T), 0, s, p, bytes, per_wg, sink); break;
    case 4: hipLaunchKernelGGL((stream_read_kernel<T, 4>), dim3(wgs), dim3(T), 0, s, p, bytes, per_wg, sink); break;
    case 8: hipLaunchKernelGGL((stream_read_kernel<T, 8>), dim3(wgs), dim3(T), 0, s, p, bytes, per_wg, sink); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// ---- issue-rate probes: one VALU instruction form, eight independent registers per
//      step, four steps per loop iteration (so the loop's own scalar instructions are
//      a small share), `iters` iterations; the host times the launch over a grid of 16
//      waves per CU and reports time per wave instruction per CU

// Instruction forms, in probe order (operands: r the register stepped, a and b two
// lane values; outputs of the pair-producing forms land in a 64-bit register pair).
#define LB_PROBE_FORMS(X)                                                   \
  X(0, "v_fmac_f32_e32 %0, %1, %2")                                         \
  X(1, "v_fma_f32 %0, %1, %2, %0")                                          \
  X(2, "v_add_f32_e32 %0, %1, %0")                                          \
  X(3, "v_mul_f32_e32 %0, %1, %0")                                          \
  X(4, "v_and_b32_e32 %0, %1, %0")                                          \
  X(5, "v_lshrrev_b32_e32 %0, 4, %0")                                       \
  X(6, "v_cvt_f32_ubyte1_e32 %0, %0")                                       \
  X(7, "v_cvt_f32_u32_e32 %0, %0")                                          \
  X(8, "v_bfe_u32 %0, %0, 4, 4")                                            \
  X(9, "v_perm_b32 %0, %1, %2, %0")                                         \
  X(10, "v_and_or_b32 %0, %1, %2, %0")                                      \
  X(11, "v_fma_mix_f32 %0, %1, %2, %0 op_sel_hi:[1,0,0]")                   \
  X(12, "v_dot4_i32_i8 %0, %1, %2, %0")                                     \
  X(13, "v_pk_add_f16 %0, %1, %0")                                          \
  X(15, "v_dot2_f32_f16 %0, %1, %2, %0")                                    \
  X(16, "v_dot2c_f32_f16_e32 %0, %1, %2")                                   \
  X(17, "v_cvt_f32_f16_e32 %0, %1")

// the 17 forms above and, as form 14, v_cvt_scalef32_pk_f32_fp4. The half-precision
// forms read a and b as pairs of finite halves (the low halves of a are 0, +-2^-7,
// +-2 or +-512; the rest are near 1.8)
constexpr int kProbeForms = 18;

template <int OP>
__global__ __launch_bounds__(512) void valu_probe_kernel(int iters, float *out) {
  // finite, normal float operands (1 + t/1024 and 0.5): the float forms never meet a
  // NaN, infinity or subnormal; the integer forms take the same bits
  uint32_t a = __float_as_uint(1.0f + (float)threadIdx.x * 0.0009765625f), b = 0x3F000000u;
  uint32_t r0 = a, r1 = a + 1, r2 = a + 2, r3 = a + 3, r4 = a + 4, r5 = a + 5, r6 = a + 6, r7 = a + 7;
  v2f p[8] = {};
  for (int i = 0; i < iters; i++) {
    if constexpr (OP == 14) {
      // the pair conversion: eight independent sources and destination pairs
#define LB_PK(J, R) asm volatile("v_cvt_scalef32_pk_f32_fp4 %0, %1, %2" : "=v"(p[J]) : "v"(R), "v"(b));
#define LB_PK8 LB_PK(0, r0) LB_PK(1, r1) LB_PK(2, r2) LB_PK(3, r3) LB_PK(4, r4) LB_PK(5, r5) LB_PK(6, r6) LB_PK(7, r7)
      LB_PK8 LB_PK8 LB_PK8 LB_PK8
#undef LB_PK8
#undef LB_PK
    } else {
#define LB_STEP(ID, INS)                                                    \
  if constexpr (OP == ID) {                                                 \
    asm volatile(INS : "+v"(r0) : "v"(a), "v"(b));                          \
    asm volatile(INS : "+v"(r1) : "v"(a), "v"(b));                          \
    asm volatile(INS : "+v"(r2) : "v"(a), "v"(b));                          \
    asm volatile(INS : "+v"(r3) : "v"(a), "v"(b));                          \
    asm volatile(INS : "+v"(r4) : "v"(a), "v"(b));                          \
    asm volatile(INS : "+v"(r5) : "v"(a), "v"(b));                          \
    asm volatile(INS : "+v"(r6) : "v"(a), "v"(b));                          \
    asm volatile(INS : "+v"(r7) : "v"(a), "v"(b));                          \
  }
      LB_PROBE_FORMS(LB_STEP)
      LB_PROBE_FORMS(LB_STEP)
      LB_PROBE_FORMS(LB_STEP)
      LB_PROBE_FORMS(LB_STEP)
#undef LB_STEP
    }
  }
  float f = __uint_as_float(r0 ^ r1 ^ r2 ^ r3 ^ r4 ^ r5 ^ r6 ^ r7);
#pragma unroll
  for (int j = 0; j < 8; j++) f += p[j].x + p[j].y;
  out[(size_t)blockIdx.x * 512 + threadIdx.x] = f;
}

template <int OP>
static void launch_probe_op(int iters, int workgroups, float *out, hipStream_t s) {
  hipLaunchKernelGGL((valu_probe_kernel<OP>), dim3(workgroups), dim3(512), 0, s, iters, out);
}

template <int... OPS>
static hipError_t launch_probe_sel(int op, int iters, int workgroups, float *out, hipStream_t s,
                                   std::integer_sequence<int, OPS...>) {
  bool found = false;
  ((op == OPS ? (launch_probe_op<OPS>(iters, workgroups, out, s), found = true) : false), ...);
  return found ? hipGetLastError() : hipErrorInvalidValue;
}

hipError_t launch_valu_probe(int op, int iters, int workgroups, float *out, hipStream_t s) {
  if (iters <= 0 || workgroups <= 0 || workgroups > 65536) return hipErrorInvalidValue;
  return launch_probe_sel(op, iters, workgroups, out, s, std::make_integer_sequence<int, kProbeForms>{});
}

int valu_probe_forms() { return kProbeForms; }

// ---- device-wide barrier probe: the cost of one barrier between all workgroups of
//      a launch, the synchronisation a persistent kernel needs between dependent
//      phases (each phase of a one-token decode step reads what every workgroup of
//      the previous phase wrote). One wave per workgroup; the host keeps the grid
//      small enough to be resident. Every wait is bounded: after `spin_limit` polls a
//      workgroup records the time-out in status[0] and returns, so the launch always
//      ends, whether or not every workgroup was resident.
//   mode 0: one counter (sync[0]); a workgroup adds 1 per round (agent-scope atomic)
//           and polls it until every workgroup's addition for the round is there
//   mode 1: one flag per workgroup (sync[64 + b], its own cache line group apart
//           from the counter); a workgroup stores its round number and polls all
//           flags, one per lane (no atomic read-modify-write: nothing serialises)
//   mode 2: mode 1 with an agent-scope release fence before the flag store and an
//           agent-scope acquire fence after the wait, which is what data written
//           before the barrier and read after it by another workgroup needs
// Counter and flags only grow, so a workgroup already in the next round never
// undoes a condition a slower one is still waiting for.
__global__ __launch_bounds__(kWave) void grid_barrier_kernel(uint32_t *sync, int rounds, int mode,
                                                             uint32_t spin_limit, uint32_t *status) {
  const uint32_t G = gridDim.x;
  const uint32_t lane = threadIdx.x;
  uint32_t *flags = sync + 64;
  for (int r = 0; r < rounds; r++) {
    const uint32_t want = (uint32_t)r + 1;
    if (mode == 2) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    if (lane == 0) {
      if (mode == 0) __hip_atomic_fetch_add(sync, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else __hip_atomic_store(flags + blockIdx.x, want, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    for (uint32_t spin = 0;; spin++) {
      bool ok = true;
      if (mode == 0) {
        ok = __hip_atomic_load(sync, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= want * G;
      } else {
        for (uint32_t i = lane; i < G; i += kWave)
          ok = ok && __hip_atomic_load(flags + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= want;
      }
      if (__all(ok)) break;
      if (spin >= spin_limit) {
        if (lane == 0) __hip_atomic_store(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (mode == 2) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
}

hipError_t launch_grid_barrier(int workgroups, int rounds, int mode, uint32_t *sync, uint32_t *status,
                               hipStream_t s) {
  if (workgroups <= 0 || workgroups > kBarrierMaxWorkgroups || rounds < 0 || rounds > 100000 || mode < 0 ||
      mode > 2)
    return hipErrorInvalidValue;
  // the counter reaches rounds * workgroups <= 1.03e8, far below 2^32
  hipError_t e = hipMemsetAsync(sync, 0, (size_t)(64 + workgroups) * 4, s);
  if (e == hipSuccess) e = hipMemsetAsync(status, 0, 4, s);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(grid_barrier_kernel, dim3(workgroups), dim3(kWave), 0, s, sync, rounds, mode,
                     (uint32_t)(1u << 16), status);
  return hipGetLastError();
}

// ---- the one-row W4A8 quantizer's division by 127 (div127, lb_device.h) on every
//      non-negative finite float32 and +inf (bit patterns 0 .. 0x7F800000) against the
//      IEEE quotient a / 127.0f, both as this device computes them. out[0] counts the
//      patterns that differ, out[1] holds the smallest of them (0xFFFFFFFF: none); the
//      init kernel sets both first. Every thread visits a fixed set of patterns
//      (grid-stride, the largest index below 0x7F800000 + stride < 2^32).
__global__ __launch_bounds__(64) void div127_init_kernel(uint32_t *out) {
  if (threadIdx.x == 0) {
    out[0] = 0u;
    out[1] = 0xFFFFFFFFu;
  }
}

__global__ __launch_bounds__(256) void div127_probe_kernel(uint32_t *out) {
  const uint32_t stride = gridDim.x * 256u;
  uint32_t bad = 0, first = 0xFFFFFFFFu;
  for (uint32_t u = blockIdx.x * 256u + threadIdx.x; u <= 0x7F800000u; u += stride) {
    const float a = __uint_as_float(u);
    if (__float_as_uint(div127(a)) != __float_as_uint(a / 127.0f)) {
      bad++;
      first = min(first, u);
    }
  }
  if (bad) {
    atomicAdd(out, bad);
    atomicMin(out + 1, first);
  }
}

hipError_t launch_div127_probe(uint32_t *out, hipStream_t s) {
  hipLaunchKernelGGL(div127_init_kernel, dim3(1), dim3(64), 0, s, out);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(div127_probe_kernel, dim3(2048), dim3(256), 0, s, out);
  return hipGetLastError();
}

__global__ __launch_bounds__(512) void empty_kernel() {}

// ---- matrix-core / VALU sharing probe: per loop iteration 8 independent
//      v_mfma_i32_16x16x64_i8 (eight accumulators), 64 independent v_fmac_f32 (eight
//      registers), or both, either one MFMA before each eight FMACs (interleaved) or
//      all eight MFMAs before the 64 FMACs (blocks). Written as inline assembly so the
//      order is exactly this; no memory access in the loop. With 256 threads per
//      workgroup and one workgroup per CU each SIMD runs one wave, with 512 two: the
//      question is whether one SIMD's matrix-core and VALU instructions overlap
//      (time of both near the larger of the two alone) or add up.
template <int V>
__global__ __launch_bounds__(512) void mfma_valu_probe_kernel(int iters, float *out) {
  v4i acc[8];
#pragma unroll
  for (int j = 0; j < 8; j++) acc[j] = v4i{0, 0, 0, 0};
  const v4i a = v4i{(int)threadIdx.x, 1, 2, 3}, b = v4i{3, 2, 1, (int)threadIdx.x};
  float r[8];
#pragma unroll
  for (int j = 0; j < 8; j++) r[j] = 1.0f + (float)threadIdx.x * 0.0009765625f + (float)j;
  const float x = 0.999f, y = 1e-7f;
  for (int i = 0; i < iters; i++) {
#pragma unroll
    for (int m = 0; m < 8; m++) {
      if constexpr (V == 0 || V == 2 || V == 3)
        asm volatile("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+v"(acc[m]) : "v"(a), "v"(b));
      if constexpr (V == 1 || V == 2) {
#pragma unroll
        for (int j = 0; j < 8; j++) asm volatile("v_fmac_f32_e32 %0, %1, %2" : "+v"(r[j]) : "v"(x), "v"(y));
      }
    }
    if constexpr (V == 3) {
#pragma unroll
      for (int m = 0; m < 8; m++)
#pragma unroll
        for (int j = 0; j < 8; j++) asm volatile("v_fmac_f32_e32 %0, %1, %2" : "+v"(r[j]) : "v"(x), "v"(y));
    }
  }
  // the last matrix-core results are read only after the longest MFMA's wait states
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  float f = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; j++) f += r[j] + (float)(acc[j].x + acc[j].y + acc[j].z + acc[j].w);
  out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = f;
}

hipError_t launch_mfma_valu_probe(int variant, int iters, int workgroups, int threads, float *out, hipStream_t s) {
  if (variant < 0 || variant > 3 || iters <= 0 || workgroups <= 0 || workgroups > 65536 ||
      (threads != 256 && threads != 512))
    return hipErrorInvalidValue;
  const dim3 g(workgroups), b(threads);
  switch (variant) {
    case 0: hipLaunchKernelGGL(mfma_valu_probe_kernel<0>, g, b, 0, s, iters, out); break;
    case 1: hipLaunchKernelGGL(mfma_valu_probe_kernel<1>, g, b, 0, s, iters, out); break;
    case 2: hipLaunchKernelGGL(mfma_valu_probe_kernel<2>, g, b, 0, s, iters, out); break;
    default: hipLaunchKernelGGL(mfma_valu_probe_kernel<3>, g, b, 0, s, iters, out); break;
  }
  return hipGetLastError();
}

hipError_t launch_empty(int workgroups, hipStream_t s) {
  if (workgroups <= 0 || workgroups > 65536) return hipErrorInvalidValue;
  hipLaunchKernelGGL(empty_kernel, dim3(workgroups), dim3(512), 0, s);
  return hipGetLastError();
}

hipError_t launch_stream_read(const void *src, size_t bytes, int workgroups, int threads, int loads, uint32_t *sink,
                              hipStream_t s) {
  if (bytes == 0 || bytes % 16 || bytes > 0xFFFFFFF0u || workgroups <= 0 || workgroups > 65536)
    return hipErrorInvalidValue;
  if (threads == 256) return launch_read_t<256>(src, (uint32_t)bytes, workgroups, loads, sink, s);
  if (threads == 512) return launch_read_t<512>(src, (uint32_t)bytes, workgroups, loads, sink, s);
  return hipErrorInvalidValue;
}

}  // namespace lbk
