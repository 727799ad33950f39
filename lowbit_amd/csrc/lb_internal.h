// Host-side launch interface between the C ABI (lb_api.hip) and the gfx950
// kernels (lb_kernels.hip). Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace lbk {

enum Fmt { F_W4A16 = 0, F_MXFP4 = 1, F_W4A8 = 2, F_W4A8Q = 3, F_W4A16G32 = 4, F_W4A8G32 = 5 };

// int4 with groups of 32 (F_W4A16G32, F_W4A8G32): the block layout of MXFP4 (byte j
// of group g holds elements 32g + j and 32g + 16 + j) with an fp32 scale and
// optional uint8 zero-point per group.
__host__ __device__ constexpr bool fmt_g32(int f) { return f == F_W4A16G32 || f == F_W4A8G32; }
__host__ __device__ constexpr int fmt_group(int f) { return fmt_g32(f) || f == F_MXFP4 ? 32 : 128; }

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
  // one-row (paced) GEMV: rows per workgroup N / grid and N % grid, divided on the host so
  // that no division runs ahead of the kernel's first loads
  int split_base = 0, split_rem = 0;
  const uint4 *x3 = nullptr;      // activations as three bf16 terms, tiled (bf16x3 path);
                                  // W4A16: two float16 terms of each row times 2^xexp[row]
  const int *xexp = nullptr;      // W4A16 batch path: each activation row's power-of-two exponent
  float *ypart = nullptr;         // bf16x3 split over K: the slices' partial outputs [ks][M][N]
  bool tiled = false;             // xq / asum in the tiled layout of the MFMA path
  bool wt16 = false;              // qw / scales / zeros / e8m0 in the MFMA tile layout (t16)
  // Decode fusions of the small-M kernels (gemv regime). Prologues (M == 1):
  const float *norm_w = nullptr;  // RMSNorm of the activation row over Kp elements, times norm_w
  float norm_eps = 0.0f;
  bool swiglu = false;            // x row is [gate (Kp) | up (Kp)]; the activation is silu(gate) * up
  // the activation row is the one-token attention output (Kp = heads x attn_d) merged
  // from attn_ns key-slice partials [heads][attn_ns][attn_d + 4] (x is not read)
  const float *attn_part = nullptr;
  int attn_ns = 0, attn_d = 0;
  // Epilogue: y = res + (x . w^T + bias); res may alias y.
  const float *bias = nullptr;    // [N]
  const float *res = nullptr;     // [M, N]
  unsigned long long *amax_key = nullptr;  // M == 1: kArgmaxSlots argmax keys of the y row, max-combined
  bool glu = false;               // rows in (gate, up) pairs; y [M, N/2] = silu(gate) * up of each pair
};

// Argmax keys are max-combined into this many slots (global wave index modulo the
// slot count), so that no single address serialises thousands of atomics.
constexpr int kArgmaxSlots = 1024;

// Prologue of a fused GEMV: 0 none, 1 RMSNorm, 2 SwiGLU, 3 attention merge.
inline int gemv_prologue(const GemmArgs &a) { return a.norm_w ? 1 : (a.swiglu ? 2 : (a.attn_part ? 3 : 0)); }

// MFMA tile layout ("t16") of int4 g128 weights, a device-private copy of the
// packed matrix in the order the int8 MFMA path consumes it. With S = ceil(N/16)
// subtiles of 16 rows and G4 = G rounded up to a multiple of 4:
//   qwt  [S][G4][64][16 B]  lane l = 16q + c of tile (s, g) holds bytes
//                           [64g + 16q, 64g + 16q + 16) of row 16s + c
//   st   [S][G4/4][16][4]   fp32 scale of row 16s + c, group 4 (g/4) + g%4
//   zt   [S][G4/4][16][4]   uint8 zero-point, same order (absent for z = 8)
// Rows past N and groups past G are zero (zero codes, scale 0, zero-point 0).
// MXFP4 weights use the same qwt order (the 16 bytes of lane (q, c) in group g are
// block 4g + q of row 16s + c) with G = ceil(Kp/128) and
//   et   [S][G4][64]        uint8 E8M0 exponent of that block (lane order)
__host__ __device__ inline int t16_groups(int Kp) { return (((Kp + 127) / 128) + 3) & ~3; }
__host__ __device__ inline size_t t16_qw_bytes(int N, int Kp) { return (size_t)((N + 15) / 16) * t16_groups(Kp) * 1024; }
__host__ __device__ inline size_t t16_group_entries(int N, int Kp) { return (size_t)((N + 15) / 16) * 16 * t16_groups(Kp); }
__host__ __device__ inline size_t t16_e8m0_bytes(int N, int Kp) { return (size_t)((N + 15) / 16) * t16_groups(Kp) * 64; }
// t16f8: the int4 tiles of the bf16 matrix-core path with each code less its
// zero-point stored as one E4M3 byte of value (code - z) 2^-9 (sign and magnitude,
// exact for |code - z| <= 15; larger differences, from zero-points above 15, are
// stored as NaN). Tile (s, g) is 2 KiB:
//   qwt8 [S][G4][2][64][16 B]  half h, lane l = 16q + c: byte b is nibble h (0 low,
//                              1 high) of byte 64g + 16q + b of row 16s + c, less z
// with st as for t16 (there is no zero-point array). Padding bytes are 0.
__host__ __device__ inline size_t t16f8_qw_bytes(int N, int Kp) { return 2 * t16_qw_bytes(N, Kp); }
hipError_t launch_repack_mxfp4_t16(const uint8_t *qw, const uint8_t *e8m0, int N, int Kp, uint8_t *qwt, uint8_t *et,
                                   hipStream_t s);
// bf16x3 path (W4A16 / MXFP4 on bf16 matrix cores, fp32-exact products): the
// activations as three bf16 terms in the A-operand tile order, and the GEMM on t16
// weights. Bytes of the split activations for M rows:
__host__ __device__ inline size_t x3_bytes(int M, int Kp) { return (size_t)((M + 15) / 16) * ((Kp + 127) / 128) * 4 * 3 * 1024; }
hipError_t launch_split3(int fmt, const float *x, int M, int Kp, uint4 *x3, hipStream_t s);
// W4A16: each activation row scaled by a power of two 2^E (its largest magnitude into
// [2^14, 2^15)) and split into two float16 terms, the second times 2^11, in the same
// tile order with two terms per slot; the exponents follow the terms at a 256-byte
// boundary. Both fit in x3_bytes(M, Kp).
__host__ __device__ inline size_t x2h_bytes(int M, int Kp) { return (size_t)((M + 15) / 16) * ((Kp + 127) / 128) * 4 * 2 * 1024; }
__host__ __device__ inline size_t x2h_exp_offset(int M, int Kp) { return (x2h_bytes(M, Kp) + 255) & ~(size_t)255; }
hipError_t launch_split2h(const float *x, int M, int Kp, uint4 *x2, int *xexp, hipStream_t s);
hipError_t launch_bf3_gemm(int fmt, const GemmArgs &a, int num_cus, hipStream_t s, bool f8 = false);
// K slices of the bf16x3 GEMM at this shape (1: no split), and the bytes of their
// partial outputs that launch_bf3_gemm needs at a.ypart when the split is taken.
int bf3_k_slices(int fmt, int M, int Kp);
size_t bf3_part_bytes(int fmt, int M, int N, int Kp);
// Whether W4A16 at this shape is faster on t16f8 weights than on t16 weights (with
// the K split the shape takes when the workspace has room for it).
bool w4a16_prefers_t16f8(int M, int N, int Kp, int num_cus);
// weight quantizers (lb_wquant.hip): fp32 [N, K] -> packed int4 with groups of `group`
// (128 or 32; mode 0 absmax, 1 signed-max, 2 asym) or MXFP4
hipError_t launch_quantize_int4(const float *w, int N, int K, int mode, int group, uint8_t *qw, float *scales,
                                uint8_t *zeros, hipStream_t s);
hipError_t launch_quantize_mxfp4(const float *w, int N, int K, uint8_t *qw, uint8_t *e8m0, hipStream_t s);
hipError_t launch_repack_int4_t16(const uint8_t *qw, const float *scales, const uint8_t *zeros, int N, int Kp,
                                  uint8_t *qwt, float *st, uint8_t *zt, hipStream_t s);
hipError_t launch_repack_int4_t16f8(const uint8_t *qw, const float *scales, const uint8_t *zeros, int N, int Kp,
                                    uint8_t *qwt8, float *st, hipStream_t s);

// Small-M VALU kernels: largest M they take and the LDS they need.
constexpr int kGemvMaxM = 4;
constexpr size_t kGemvLdsLimit = 60 * 1024;  // dynamic LDS, leaving room for static scratch
size_t gemv_lds_bytes(int fmt, int M, int Kp);
bool gemv_eligible(int fmt, int M, int Kp);

// The instantiation and grid a small-M launch takes for a shape (the test hook behind
// lbd_gemm_plan); with a non-null plan, launch_gemv fills it and launches nothing.
struct GemvPlan {
  int workgroups = 0, rows_per_wave = 0, rows_held = 0, chunks_per_lane = 0, two_rows_per_load = 0, act_rows = 0;
  int k_slices = 1;  // slices each weight row is cut into across waves (rows past 4096 elements)
};
hipError_t launch_gemv(int fmt, const GemmArgs &a, int num_cus, hipStream_t s, GemvPlan *plan = nullptr);
// Workgroups of a small-M kernel (`threads` per workgroup, `lds` bytes of dynamic
// LDS) that fit on one CU at once; asked of the runtime once per kernel and size.
int gemv_wg_per_cu(const void *kern, size_t lds, int threads = 512);
// the group-32 instantiations of the small-M kernels (lb_gemv_g32.hip)
hipError_t launch_gemv_g32(int fmt, const GemmArgs &a, int num_cus, size_t lds, hipStream_t s, GemvPlan *plan);
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
// Plain streaming read of `bytes` (multiple of 16, below 4 GiB) by `workgroups` groups
// of `threads` (256 or 512) threads with `loads` (1, 2, 4, 8) 16-byte loads in flight
// per thread (lb_probe.hip); `sink` is one device dword it almost never writes.
hipError_t launch_stream_read(const void *src, size_t bytes, int workgroups, int threads, int loads, uint32_t *sink,
                              hipStream_t s);
// VALU issue-rate probe `op` (0 .. valu_probe_forms() - 1), `iters` iterations of 32
// instructions per thread (eight independent registers, four steps), workgroups of 512
// threads; out[workgroups * 512].
hipError_t launch_valu_probe(int op, int iters, int workgroups, float *out, hipStream_t s);
int valu_probe_forms();
// a kernel that does nothing, workgroups of 512 threads
hipError_t launch_empty(int workgroups, hipStream_t s);
// Matrix-core / VALU sharing probe: variant 0 MFMA only, 1 VALU only, 2 both
// interleaved, 3 both in blocks; `threads` 256 or 512; out: workgroups * threads floats.
hipError_t launch_mfma_valu_probe(int variant, int iters, int workgroups, int threads, float *out, hipStream_t s);
// div127 against a / 127.0f on every non-negative finite float32 and +inf: out[0] the
// number that differ, out[1] the smallest differing bit pattern (0xFFFFFFFF: none)
hipError_t launch_div127_probe(uint32_t *out, hipStream_t s);
// Device-wide barrier probe (lb_probe.hip): `rounds` barriers between `workgroups`
// (1 .. kBarrierMaxWorkgroups) one-wave workgroups, `mode` 0 (one atomic counter), 1
// (a flag per workgroup) or 2 (flags with agent-scope release / acquire fences).
// Clears sync[64 + workgroups] and status[1] on the stream first (not for capture);
// status[0] becomes 1 if a wait timed out.
constexpr int kBarrierMaxWorkgroups = 1024;
hipError_t launch_grid_barrier(int workgroups, int rounds, int mode, uint32_t *sync, uint32_t *status,
                               hipStream_t s);

// Decoder-layer kernels (lb_model.hip).
hipError_t launch_embed(const float *table, int vocab, int hidden, const int32_t *tok, int T, float *x, hipStream_t s);
hipError_t launch_rmsnorm(const float *x, const float *w, int T, int hidden, float eps, float *y, hipStream_t s);
hipError_t launch_qkv_rope(float *qkv, const float *bias, int T, int H, int KV, int D, const float *cosT,
                           const float *sinT, const int32_t *pos, int max_pos, float *kc, float *vc, int cap,
                           hipStream_t s);
hipError_t launch_attention(const float *q, int qstride, const float *kc, const float *vc, int T, int H, int KV, int D,
                            const int32_t *pos, int cap, float *out, hipStream_t s);
hipError_t launch_swiglu(const float *gu, int T, int I, float *out, hipStream_t s);
hipError_t launch_swiglu_pairs(const float *gu, int T, int I, float *out, hipStream_t s);
hipError_t launch_add(float *x, const float *y, size_t n, hipStream_t s);
hipError_t launch_argmax(const float *v, int n, int32_t *tok, int32_t *pos, int inc, int32_t *hist, int hist_len,
                         hipStream_t s);
hipError_t launch_argmax_finalize(unsigned long long *key, int32_t *tok, int32_t *pos, int inc, int32_t *hist,
                                  int hist_len, hipStream_t s);
// One-token attention with the rotary embedding and the KV-cache write folded in.
// With a workspace and a cache of at least kAttnSliceMinCap positions, each query
// head's keys are cut into slices of one wave round (attn_slice_keys), at most
// kAttnMaxSplit per head, whose partials [H][slices][D + 4] floats a second kernel
// (or a fused GEMV's attention-merge prologue, up to kAttnMaxFusedSlices slices)
// merges; otherwise one workgroup per query head (work may be null).
constexpr int kAttnMaxGroup = 16;     // query heads per KV head
constexpr int kAttnMaxSplit = 32;     // key slices per head
constexpr int kAttnMaxFusedSlices = 8;  // slices a fused GEMV's prologue merges
constexpr int kAttnSliceMinCap = 1024;
// Keys per slice: one wave round of 8 loads per lane (2048 / D keys) where 8 such
// slices hold the cache (more workgroups, each one shorter), else 16 (4096 / D).
inline int attn_slice_keys(int D, int cap) {
  const int k8 = 32 * 64 / D;
  return (cap + k8 - 1) / k8 <= kAttnMaxFusedSlices ? k8 : 2 * k8;
}
inline int attn_slices(int D, int cap) {
  const int kb = attn_slice_keys(D, cap);
  const int n = (cap + kb - 1) / kb;
  return n < kAttnMaxSplit ? n : kAttnMaxSplit;
}
inline size_t attn_work_bytes(int H, int D, int cap) {
  return (size_t)H * attn_slices(D, cap) * (D + 4) * sizeof(float);
}
hipError_t launch_attention_decode(const float *qkv, int H, int KV, int D, const float *cosT, const float *sinT,
                                   const int32_t *pos, int max_pos, float *kc, float *vc, int cap, float *out,
                                   float *work, hipStream_t s);
hipError_t launch_attention_slices(const float *qkv, int H, int KV, int D, const float *cosT, const float *sinT,
                                   const int32_t *pos, int max_pos, float *kc, float *vc, int cap, float *part,
                                   hipStream_t s);
hipError_t launch_attention_merge(const float *part, int H, int D, const int32_t *pos, int cap, float *out,
                                  hipStream_t s);

}  // namespace lbk
