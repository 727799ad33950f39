/*
 * lowbit_hip: fused dequantize + GEMM for low-bit weights on AMD Instinct MI355X (gfx950).
 *
 * C ABI of liblowbit_hip.so. Every GEMM computes  Y[M,N] = X[M,Kp] . W[N,Kp]^T
 * (nn.Linear convention). Kp is the padded reduction length: a multiple of 128
 * for the int4 formats, of 32 for MXFP4; callers pad X with zeros.
 *
 * Packed weight layouts (row n of W is Kp/2 contiguous bytes):
 *   int4, group 128 : group g = bytes [64g, 64g+64); byte j holds element 128g+j
 *                     (low nibble) and 128g+64+j (high nibble). value = (q - z) * s,
 *                     q in 0..15, s = scales[n,g] (fp32), z = zeros[n,g] or 8
 *                     when zeros == NULL.
 *   MXFP4, block 32 : block b = bytes [16b, 16b+16); byte j holds element 32b+j
 *                     (low nibble) and 32b+16+j (high nibble); OCP E2M1 codes,
 *                     value = e2m1(q) * 2^(e8m0[n,b] - 127) (e8m0 0 -> 2^-127,
 *                     255 -> NaN).
 *   Same layouts as the reference, src/lowbit/csrc/lowbit.h:9-19.
 *
 * Three families of entry points:
 *   lb_*    host pointers, synchronous: the exact signatures of the reference ABI
 *           (src/lowbit/csrc/lowbit.h:95-123). Inputs are copied to the device,
 *           the kernel runs, y is copied back before return.
 *   lbd_*   device pointers, asynchronous on `stream` (a hipStream_t, NULL = the
 *           null stream). For callers that keep weights and activations resident
 *           in HBM. Nothing is copied; the call returns after the launch.
 *   lb_dev_*, lb_stream_*, lb_event_*: minimal device-memory, stream and event
 *           plumbing so that a caller without its own HIP runtime bindings (the
 *           ctypes layer) can use the lbd_* family.
 *
 * Return codes: >= 0 success (the id of the path that ran, LB_ISA_*), < 0 error.
 * These follow the reference (src/lowbit/csrc/dispatch.c:160,205-208,279):
 *   -1 bad shape (M, N or Kp <= 0, or Kp not a multiple of the block),
 *   -2 tile parameters that name no compiled micro-tile (lb_params.mr/nr),
 *   -3 allocation failure, -4 feature unavailable (no device / AMX entry points),
 *   plus -5 HIP runtime error and -6 bad argument (NULL pointer, bad isa).
 * lb_last_error() gives a message for the last failure on the calling thread.
 *
 * Threading: every host thread gets its own stream and staging buffers, so the
 * lb_* entry points may be called concurrently from several threads.
 */
#ifndef LOWBIT_HIP_H
#define LOWBIT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LB_GROUP 128  /* int4 group size (elements) */
#define LB_MXBLOCK 32 /* MXFP4 block size (elements) */
#define LB_G32 32     /* the group size of the group-32 int4 entry points */

/* Path ids, returned by the GEMMs like the reference returns its ISA id
 * (src/lowbit/csrc/dispatch.c:202). The reference's CPU ids 0..2 (scalar, avx2,
 * avx512) are accepted as requests and mean "auto": there are no CPU tiers. */
#define LB_ISA_GFX950 16      /* VALU decode kernels (small M) */
#define LB_ISA_GFX950_MFMA 17 /* matrix-core kernels (M >= 16 or large M*K) */

#define LB_ERR_SHAPE -1
#define LB_ERR_TILE -2
#define LB_ERR_ALLOC -3
#define LB_ERR_UNAVAILABLE -4
#define LB_ERR_HIP -5
#define LB_ERR_ARG -6

/* Dispatch parameters; zero or negative fields mean "default".
 * Same struct as the reference (src/lowbit/csrc/lowbit.h:37-45). `isa` requests a
 * path (-1 auto, LB_ISA_GFX950, LB_ISA_GFX950_MFMA; a VALU request that the shape
 * cannot use is clamped to MFMA, as the reference clamps its ISA). mr/nr must name
 * one of the reference's micro-tiles (1,2,4,8 x 1,2,4 minus 8x4) or be 0, else -2;
 * nb/kb/order/nthreads are accepted and have no GPU meaning. */
typedef struct {
    int isa;
    int mr;
    int nr;
    int nb;
    int kb;
    int order;
    int nthreads;
} lb_params;

/* ---- library / device information (src/lowbit/csrc/lowbit.h:95-103) ---- */
int lb_version(void);
/* best path the hardware supports: LB_ISA_GFX950_MFMA on a gfx950 device, -4 without one
 * (replaces lowbit.h:96 lb_cpu_isa) */
int lb_cpu_isa(void);
/* same after the LOWBIT_ISA environment cap ("gfx950" limits GEMMs to the VALU
 * kernels; replaces lowbit.h:97 lb_active_isa) */
int lb_active_isa(void);
int lb_has_vnni(void);    /* 0: no CPU VNNI path in this library (lowbit.h:98) */
int lb_has_openmp(void);  /* 0 (lowbit.h:99) */
int lb_max_threads(void); /* 1: host threads are not used for compute (lowbit.h:100) */
/* path a GEMM kind (0 w4a16, 1 mxfp4, 2 w4a8) runs with for a request; mirrors
 * lowbit.h:102 lb_effective_isa. The shape-dependent regime is reported by the
 * GEMM's return value. */
int lb_effective_isa(int kind, int requested);
/* device name, compute units and LDS bytes per workgroup of the current device */
int lb_device_info(char *name, int name_len, int *compute_units, int *lds_bytes);
const char *lb_last_error(void);
/* return code of the last lb_* / lbd_* call on this thread (lets callers of the
 * void lb_quant_act_int8 see a failure) */
int lb_last_status(void);

/* ---- GEMMs, host pointers (src/lowbit/csrc/lowbit.h:105-123) ---- */
int lb_gemm_w4a16(const float *x, int M, int Kp, const uint8_t *qw,
                  const float *scales, const uint8_t *zeros, int N, float *y,
                  const lb_params *p);
int lb_gemm_mxfp4(const float *x, int M, int Kp, const uint8_t *qw,
                  const uint8_t *e8m0, int N, float *y, const lb_params *p);
/* x is fp32; the per-token int8 quantization runs on the device inside the call */
int lb_gemm_w4a8(const float *x, int M, int Kp, const uint8_t *qw,
                 const float *scales, const uint8_t *zeros, int N, float *y,
                 const lb_params *p);
/* activations already quantized: xq [M,Kp], xs [M], asum [M,Kp/128] */
int lb_gemm_w4a8_q(const int8_t *xq, const float *xs, const int32_t *asum,
                   int M, int Kp, const uint8_t *qw, const float *scales,
                   const uint8_t *zeros, int N, float *y, const lb_params *p);
/* per-token symmetric int8 quantization, bit-identical to the reference
 * (src/lowbit/csrc/dispatch.c:231-257); runs on the device */
void lb_quant_act_int8(const float *x, int M, int Kp, int8_t *xq, float *xs,
                       int32_t *asum);
/* exact int32 group accumulators out[m,n,g] = sum_{k in g} (q - z) * xq (test hook,
 * src/lowbit/csrc/dispatch.c:288-305). isa selects the integer path that produces
 * them: -1 or LB_ISA_GFX950 the VALU dot4 path, LB_ISA_GFX950_MFMA the int8 MFMA path. */
int lb_w4a8_group_acc(const int8_t *xq, const int32_t *asum, int M, int Kp,
                      const uint8_t *qw, const uint8_t *zeros, int N,
                      int32_t *out, int isa);

/* ---- GEMMs, device pointers, asynchronous on `stream` (no reference counterpart:
 *      the reference's buffers are host memory; these are what a device-resident
 *      caller binds instead of lowbit.h:105-123) ---- */
int lbd_gemm_w4a16(const float *x, int M, int Kp, const uint8_t *qw,
                   const float *scales, const uint8_t *zeros, int N, float *y,
                   const lb_params *p, void *stream);
int lbd_gemm_mxfp4(const float *x, int M, int Kp, const uint8_t *qw,
                   const uint8_t *e8m0, int N, float *y, const lb_params *p,
                   void *stream);
/* workspace: device scratch of at least lbd_w4a8_workspace_bytes(M, Kp) bytes for the
 * quantized activations, or NULL to use a buffer the library keeps per thread
 * and device (grown on demand; calls on one thread must then not overlap on
 * different streams). */
int lbd_gemm_w4a8(const float *x, int M, int Kp, const uint8_t *qw,
                  const float *scales, const uint8_t *zeros, int N, float *y,
                  const lb_params *p, void *workspace, size_t workspace_bytes,
                  void *stream);
size_t lbd_w4a8_workspace_bytes(int M, int Kp);
int lbd_gemm_w4a8_q(const int8_t *xq, const float *xs, const int32_t *asum,
                    int M, int Kp, const uint8_t *qw, const float *scales,
                    const uint8_t *zeros, int N, float *y, const lb_params *p,
                    void *stream);
int lbd_quant_act_int8(const float *x, int M, int Kp, int8_t *xq, float *xs,
                       int32_t *asum, void *stream);
int lbd_w4a8_group_acc(const int8_t *xq, const int32_t *asum, int M, int Kp,
                       const uint8_t *qw, const uint8_t *zeros, int N,
                       int32_t *out, int isa, void *stream);

/* regime (LB_ISA_GFX950 or LB_ISA_GFX950_MFMA) an lbd_gemm_* of kind 0 = W4A16,
 * 1 = MXFP4, 2 = W4A8 with this shape and lb_params runs in (no reference
 * counterpart; the reference's effective ISA does not depend on the shape), or the
 * error such a call would return for its shape or lb_params (LB_ERR_SHAPE, or
 * LB_ERR_TILE for a micro-tile the reference does not compile) */
int lbd_gemm_path(int kind, int M, int Kp, const lb_params *p);
/* The regime and, on the small-M (VALU) path, the kernel configuration an lbd_gemm_*
 * of kind 0 = W4A16, 1 = MXFP4, 2 = W4A8 with this shape takes on the current device
 * (a test and measurement hook, no reference counterpart: the reference's GEMMs
 * report only their ISA). Fields past `path` are 0 on the matrix-core path. */
typedef struct {
  int path;              /* LB_ISA_GFX950 or LB_ISA_GFX950_MFMA */
  int workgroups;        /* grid of the small-M launch */
  int rows_per_wave;     /* weight rows each wave owns */
  int rows_held;         /* weight rows each wave has in flight at once */
  int chunks_per_lane;   /* 16-byte chunks per lane per weight row */
  int two_rows_per_load; /* 1 where each wave load covers two short rows */
  int act_rows;          /* activation rows per launch */
  int k_slices;          /* slices of 4096 elements each row is cut into, one wave each */
} lbd_plan;
int lbd_gemm_plan(int kind, int M, int N, int Kp, const lb_params *p, lbd_plan *out);

/* ---- MFMA tile layout ("t16") of int4 g128 weights (no reference counterpart:
 *      a device-private copy of an Int4Weights matrix, src/lowbit/formats.py:56-87,
 *      in the order the int8 matrix cores consume it, so that every 16-byte weight
 *      load of a wave reads one contiguous 1 KiB tile; the role pack_amx plays for
 *      the reference's AMX path, src/lowbit/formats.py:253-293). With S = ceil(N/16)
 *      subtiles of 16 rows and G4 = Kp/128 rounded up to a multiple of 4:
 *        qwt [S][G4][64][16 B]: lane 16q + c of tile (s, g) holds bytes
 *                               [64g + 16q, 64g + 16q + 16) of row 16s + c
 *        st  [S][G4/4][16][4]   fp32 scale of row 16s + c, group g (entry g % 4)
 *        zt  [S][G4/4][16][4]   uint8 zero-point, same order (NULL: z = 8)
 *      Rows past N and groups past Kp/128 are zero. ---- */
/* sizes in bytes of the three arrays; returns 0 or LB_ERR_SHAPE */
int lbd_int4_t16_bytes(int N, int Kp, size_t *qwt_bytes, size_t *st_bytes,
                       size_t *zt_bytes);
/* fills qwt / st / zt (zt only when zeros != NULL) from row-major device arrays */
int lbd_repack_int4_t16(const uint8_t *qw, const float *scales,
                        const uint8_t *zeros, int N, int Kp, uint8_t *qwt,
                        float *st, uint8_t *zt, void *stream);
/* y = x . w^T as lbd_gemm_w4a8 (same workspace contract), weights in the t16
 * layout; always the int8 matrix-core path (returns LB_ISA_GFX950_MFMA) */
int lbd_gemm_w4a8_t16(const float *x, int M, int Kp, const uint8_t *qwt,
                      const float *st, const uint8_t *zt, int N, float *y,
                      const lb_params *p, void *workspace,
                      size_t workspace_bytes, void *stream);
/* lbd_gemm_w4a8_t16 without allocation (no reference counterpart: for callers that
 * cannot allocate device memory, such as code under HIP graph capture and serving
 * loops that forbid hipMalloc). The quantized activations live in a scratch array of
 * lbd_noalloc_scratch_bytes() = 8 MiB that the library keeps on each device for the
 * life of the process, so lbd_w4a8_workspace_bytes(M, Kp) must not exceed it (else
 * LB_ERR_SHAPE; M * Kp up to about 8 million). Every call on one device shares that
 * array: calls that overlap on one device (other streams, other threads) race and
 * must be ordered by the caller. Same results as lbd_gemm_w4a8_t16, bit for bit. */
size_t lbd_noalloc_scratch_bytes(void);
int lbd_gemm_w4a8_t16_noalloc(const float *x, int M, int Kp, const uint8_t *qwt, const float *st,
                              const uint8_t *zt, int N, float *y, const lb_params *p, void *stream);
/* y = x . w^T as lbd_gemm_w4a16, weights in the t16 layout, on float16 matrix
 * cores within the reference's float32 bound (src/lowbit/csrc/kern_scalar.c:10-47,
 * tests/test_kernels.py:108-116): each row of x is scaled by a power of two and
 * split into two float16 terms (in `workspace`, lbd_bf16x3_workspace_bytes(M, Kp)
 * bytes, 256-byte aligned, or NULL for the per-thread buffer), 22 significant bits
 * of every element within 2^17 of its row's largest magnitude; every weight q - z is
 * exact in float16 and the sums are float32. Always the matrix-core path. */
int lbd_gemm_w4a16_t16(const float *x, int M, int Kp, const uint8_t *qwt,
                       const float *st, const uint8_t *zt, int N, float *y,
                       const lb_params *p, void *workspace,
                       size_t workspace_bytes, void *stream);
size_t lbd_bf16x3_workspace_bytes(int M, int Kp);
/* Workspace bytes for the bf16x3 GEMMs (lbd_gemm_w4a16_t16 / _t16f8, kind 0, and
 * lbd_gemm_mxfp4_t16, kind 1) that also lets them split K over the workgroups of a
 * column where the shape gains (rows of at least 8192 elements): the split
 * activations, then the slices' partial outputs, added by one more launch in slice
 * order. A workspace of this size (or NULL) takes the split, one of
 * lbd_bf16x3_workspace_bytes the unsplit GEMM; both meet the same bound, not the
 * same bits. Equals lbd_bf16x3_workspace_bytes rounded up to 256 where no split is
 * taken; 0 for an invalid argument. (No reference counterpart: the reference's
 * GEMMs take no workspace.) */
size_t lbd_bf16x3_workspace_bytes_split(int kind, int M, int N, int Kp);
/* ---- "t16f8": int4 g128 weights for lbd_gemm_w4a16 on the matrix cores with the
 *      zero-point folded in (no reference counterpart: a device-private copy of an
 *      Int4Weights matrix, src/lowbit/formats.py:56-87, converted two operands per
 *      instruction). Each code less its group's zero-point
 *      (z = 8 when zeros is NULL) is one E4M3 byte of value (code - z) 2^-9: sign
 *      and magnitude, exact for |code - z| <= 15, which holds for every zero-point
 *      the reference's packer writes (0-15, src/lowbit/formats.py:122); a larger
 *      difference is stored as NaN, so results are NaN rather than wrong.
 *        qwt8 [S][G4][2][64][16 B]  half h, lane 16q + c of tile (s, g): byte b is
 *                                   nibble h (0 low, 1 high) of byte 64g + 16q + b
 *                                   of row 16s + c, less z
 *        st   as for t16
 *      Rows past N and groups past Kp/128 are zero bytes. ---- */
int lbd_int4_t16f8_bytes(int N, int Kp, size_t *qwt8_bytes, size_t *st_bytes);
int lbd_repack_int4_t16f8(const uint8_t *qw, const float *scales,
                          const uint8_t *zeros, int N, int Kp, uint8_t *qwt8,
                          float *st, void *stream);
/* 1 when lbd_gemm_w4a16_t16f8 is expected to be faster than lbd_gemm_w4a16_t16 at
 * this shape on the current device (enough weight subtiles per workgroup to hide
 * the t16f8 layout's doubled weight bytes, counted for the launch with the K split a
 * workspace of lbd_bf16x3_workspace_bytes_split bytes, or NULL, gives), else 0; or
 * LB_ERR_SHAPE */
int lbd_w4a16_prefers_t16f8(int M, int N, int Kp);
/* y = x . w^T as lbd_gemm_w4a16_t16 (same workspace contract, same results bit for
 * bit) on t16f8 weights; always the matrix-core path */
int lbd_gemm_w4a16_t16f8(const float *x, int M, int Kp, const uint8_t *qwt8,
                         const float *st, int N, float *y, const lb_params *p,
                         void *workspace, size_t workspace_bytes, void *stream);
/* MXFP4 in the t16 order: qwt as above (lane 16q + c of tile (s, g) holds block
 * 4g + q of row 16s + c), et [S][G4][64] the E8M0 byte of that block (G = ceil(Kp/128)) */
int lbd_mxfp4_t16_bytes(int N, int Kp, size_t *qwt_bytes, size_t *et_bytes);
int lbd_repack_mxfp4_t16(const uint8_t *qw, const uint8_t *e8m0, int N, int Kp,
                         uint8_t *qwt, uint8_t *et, void *stream);
/* y = x . w^T as lbd_gemm_mxfp4 on t16 weights, the bf16 matrix-core path of
 * lbd_gemm_w4a16_t16 (block scales 2^(e - 127) exact; E8M0 255 gives NaN) */
int lbd_gemm_mxfp4_t16(const float *x, int M, int Kp, const uint8_t *qwt,
                       const uint8_t *et, int N, float *y, const lb_params *p,
                       void *workspace, size_t workspace_bytes, void *stream);

/* ---- weight quantizers on the device: fp32 w [N, K] row-major (device memory)
 *      -> the public packed formats, byte for byte what the host packers write
 *      (quantize_int4 / quantize_mxfp4, src/lowbit/formats.py:90-142, 197-212) for
 *      finite weights. K is padded to the block; padded elements decode to 0. ---- */
/* int4 g128 -> qw [N, Kp/2], scales [N, Kp/128], zeros [N, Kp/128] (asym only; NULL
 * otherwise). asym: s = (max(w,0) - min(w,0)) / 15 with a zero point; signed_max: s =
 * m / -8 for the element m of largest magnitude; neither: s = max|w| / 7 */
int lbd_quantize_int4(const float *w, int N, int K, int asym, int signed_max, uint8_t *qw,
                      float *scales, uint8_t *zeros, void *stream);
/* MXFP4 -> qw [N, Kp/2], e8m0 [N, Kp/32]; Kp = K rounded up to 32 */
int lbd_quantize_mxfp4(const float *w, int N, int K, uint8_t *qw, uint8_t *e8m0,
                       void *stream);

/* ---- int4 with groups of 32 (no lowbit.h counterpart: the reference ships group 128
 *      only and names groups of 32 as its main quality lever, README.md:300-304,
 *      511-512). Layout of each row: group g is bytes [16g, 16g+16); byte j holds
 *      element 32g+j (low nibble) and 32g+16+j (high nibble), the arrangement of the
 *      MXFP4 blocks; value = (q - z) * s with fp32 scales[N, Kp/32] and uint8
 *      zeros[N, Kp/32] (NULL: z = 8). Kp is a multiple of 32, at most 14336 for
 *      W4A16 (fp32 activations staged in LDS) and 16384 for W4A8. ---- */
/* y = x . w^T, fp32 activations and accumulation (the W4A16 semantics); device
 * pointers, asynchronous on `stream`. Any M: the small-M kernels run on slices of
 * at most four rows (there is no matrix-core path for groups of 32). */
int lbd_gemm_w4a16_g32(const float *x, int M, int Kp, const uint8_t *qw, const float *scales,
                       const uint8_t *zeros, int N, float *y, void *stream);
/* W4A8: x quantized per token to int8 inside the call (the reference's quantizer),
 * exact int32 sums per group of 32, then s and the token scale in fp32 */
int lbd_gemm_w4a8_g32(const float *x, int M, int Kp, const uint8_t *qw, const float *scales,
                      const uint8_t *zeros, int N, float *y, void *stream);
/* lbd_quantize_int4 with groups of 32: scales / zeros [N, Kp/32], Kp = K rounded up to 32 */
int lbd_quantize_int4_g32(const float *w, int N, int K, int asym, int signed_max, uint8_t *qw,
                          float *scales, uint8_t *zeros, void *stream);

/* ---- decoder-layer operations for a device-resident decoder (no lowbit.h
 *      counterpart: the building blocks of the reference's numpy model,
 *      src/lowbit/model.py:190-230 and 353-435, on the device; fp32 [T, width]
 *      row-major activations, asynchronous on `stream`). `pos` and `tok` are device
 *      int32: kernels read the decode position from `pos`, so a decode step is a
 *      fixed launch sequence a HIP graph can replay. ---- */
/* x[t] = table[tok[t]] (ids clamped into [0, vocab)) */
int lbd_embed(const float *table, int vocab, int hidden, const int32_t *tok, int T,
              float *x, void *stream);
/* y = x / sqrt(mean(x^2) + eps) * w per row (model.py:190-192) */
int lbd_rmsnorm(const float *x, const float *w, int T, int hidden, float eps,
                float *y, void *stream);
/* qkv [T, (H + 2 KV) D]: + bias (NULL: none), rotary embedding of q and k at
 * position *pos + t from cos/sin [max_pos, D/2] ("rotate_half", model.py:201-210),
 * q left in place, k and v written to the caches [KV, cap, D]; D in {32, 64, 128} */
int lbd_qkv_rope(float *qkv, const float *bias, int T, int H, int KV, int D,
                 const float *cos_table, const float *sin_table, const int32_t *pos,
                 int max_pos, float *k_cache, float *v_cache, int cap, void *stream);
/* out [T, H D] = causal grouped-query attention of the q rows (row stride qstride
 * floats) over cache positions 0 .. *pos + t (model.py:353-378); cap <= 16000 */
int lbd_attention(const float *q, int qstride, const float *k_cache,
                  const float *v_cache, int T, int H, int KV, int D, const int32_t *pos,
                  int cap, float *out, void *stream);
/* out [T, I] = silu(gu[:, :I]) * gu[:, I:] (model.py:213, 416-417) */
int lbd_swiglu(const float *gu, int T, int I, float *out, void *stream);
/* out [T, I] = silu(gu[:, 2i]) * gu[:, 2i + 1]: the same operation on gate/up rows
 * stored in pairs (the layout the glu epilogue of the fused GEMVs consumes) */
int lbd_swiglu_pairs(const float *gu, int T, int I, float *out, void *stream);
/* x += y over n floats (the residual adds) */
int lbd_add(float *x, const float *y, size_t n, void *stream);
/* tok[0] = numpy's argmax of v[0..n) (the first NaN if any, else the first maximum);
 * with pos != NULL also hist[*pos + inc] = tok[0] (inside [0, hist_len)) and
 * *pos += inc */
int lbd_argmax(const float *v, int n, int32_t *tok, int32_t *pos, int inc,
               int32_t *hist, int hist_len, void *stream);

/* ---- fused decode GEMVs (no lowbit.h counterpart: the reference's decoder runs a
 *      Linear as GEMM + bias in numpy, src/lowbit/model.py:120-124, with RMSNorm,
 *      SwiGLU and the residual adds as separate numpy steps, model.py:190-192,
 *      213, 398-431; a device-resident decode step folds them into the small-M
 *      kernels so each linear layer is one launch). Same operands and arithmetic
 *      as lbd_gemm_w4a16 / lbd_gemm_mxfp4 / lbd_gemm_w4a8 (W4A8 quantizes the
 *      prologue's output per token), small-M kernels only: M <= 4 and Kp within
 *      their limit (lbd_gemm_path gives LB_ISA_GFX950), else LB_ERR_SHAPE. ---- */
typedef struct {
  /* prologue, M == 1 only, at most one of the two:
   *   norm_w != NULL: x <- x * (1 / sqrt(mean(x^2) + norm_eps)) * norm_w, the mean
   *                   over the Kp elements of the row (model.py:190-192)
   *   swiglu != 0:    the x row holds 2 Kp floats [gate | up] and the activation
   *                   is silu(gate) * up, silu(g) = g / (1 + exp(-g)) (model.py:213) */
  const float *norm_w;
  float norm_eps;
  int swiglu;
  /* epilogue: y[m, n] = residual[m, n] + ((x . w^T)[m, n] + bias[n]); NULL skips a
   * term; residual may be y itself (each element is read before it is written) */
  const float *bias;
  const float *residual;
  /* M == 1: each finished y[0, n] is folded with 64-bit atomic max operations into
   * argmax_key[0 .. LBD_ARGMAX_SLOTS), as a key ordered as numpy's argmax (first NaN,
   * else first maximum); the slots must be 0 before the call (lbd_argmax_finalize
   * reads the index and clears them). 8-byte aligned device memory. */
  unsigned long long *argmax_key;
  /* glu != 0: the weight rows come in pairs (row 2p the gate, row 2p + 1 the up
   * projection of output p; N even) and y [M, N/2] receives y[m, p] = silu(g) * u of
   * the pair's outputs g, u (bias added; model.py:213), computed once per output in
   * the epilogue instead of once per workgroup in the next GEMV's SwiGLU prologue.
   * Excludes residual and argmax_key. */
  int glu;
  /* attention-merge prologue (M == 1, no other prologue): the activation row is the
   * one-token attention output, Kp = heads x attn_head_dim <= 2048, merged from the
   * key-slice partials that lbd_attention_slices wrote to attn_part for a cache of
   * attn_cap positions (at most 8 slices: attn_cap <= 8 * 4096 / attn_head_dim);
   * the result is bit for bit lbd_attention_merge's. x is not read (may be NULL). */
  const float *attn_part;
  int attn_cap;
  int attn_head_dim;
} lbd_fusion;
#define LBD_ARGMAX_SLOTS 1024
int lbd_gemv_w4a16_fused(const float *x, int M, int Kp, const uint8_t *qw, const float *scales,
                         const uint8_t *zeros, int N, float *y, const lbd_fusion *f, void *stream);
int lbd_gemv_mxfp4_fused(const float *x, int M, int Kp, const uint8_t *qw, const uint8_t *e8m0,
                         int N, float *y, const lbd_fusion *f, void *stream);
int lbd_gemv_w4a8_fused(const float *x, int M, int Kp, const uint8_t *qw, const float *scales,
                        const uint8_t *zeros, int N, float *y, const lbd_fusion *f, void *stream);
/* tok[0] = the index held by the largest of the LBD_ARGMAX_SLOTS keys (0 if all are
 * 0), then as lbd_argmax: with pos != NULL hist[*pos + inc] = tok[0] (inside
 * [0, hist_len)) and *pos += inc; finally every slot is cleared for the next step */
int lbd_argmax_finalize(unsigned long long *key, int32_t *tok, int32_t *pos, int inc,
                        int32_t *hist, int hist_len, void *stream);
/* One token at position *pos: lbd_qkv_rope (without the bias, which the qkv GEMV's
 * epilogue adds) and lbd_attention with T = 1 in one launch, one workgroup per query
 * head (model.py:353-378). qkv [(H + 2 KV) D] is read only; k and v are written to
 * the caches; out [H D]. H / KV <= 16, D in {32, 64, 128}, cap <= 16000; qkv, the
 * tables and the caches 16-byte aligned. */
int lbd_attention_decode(const float *qkv, int H, int KV, int D, const float *cos_table,
                         const float *sin_table, const int32_t *pos, int max_pos,
                         float *k_cache, float *v_cache, int cap, float *out, void *stream);
/* The same with a workspace for long caches: with work != NULL and cap >= 1024, each
 * query head's keys are cut into slices of 4096 / D keys on one-wave workgroups (at
 * most 32 per head) and a second launch merges their partial sums from `work`, so a
 * head's keys stream through many compute units; shorter caches (or work == NULL)
 * take lbd_attention_decode's one-workgroup-per-head kernel. work: device memory of
 * lbd_attention_decode_work_bytes(H, D, cap) bytes, 16-byte aligned (out too); calls
 * sharing it must be ordered (one stream). */
size_t lbd_attention_decode_work_bytes(int H, int D, int cap);
/* The two halves of the key-slice path, for callers that merge elsewhere (the
 * attention-merge prologue of the fused GEMVs): lbd_attention_slices rotates, writes
 * the caches and stores every slice's partial to `part` (slices of 2048 / D keys
 * where 8 of them hold the cache, else 4096 / D, at most 32 per head;
 * lbd_attention_decode_work_bytes(H, D, cap) bytes; slices past the keys in use
 * store empty partials); lbd_attention_merge combines them into out. */
int lbd_attention_slices(const float *qkv, int H, int KV, int D, const float *cos_table,
                         const float *sin_table, const int32_t *pos, int max_pos,
                         float *k_cache, float *v_cache, int cap, float *part,
                         size_t part_bytes, void *stream);
int lbd_attention_merge(const float *part, size_t part_bytes, int H, int D, const int32_t *pos,
                        int cap, float *out, void *stream);
int lbd_attention_decode_ws(const float *qkv, int H, int KV, int D, const float *cos_table,
                            const float *sin_table, const int32_t *pos, int max_pos,
                            float *k_cache, float *v_cache, int cap, float *out, void *work,
                            size_t work_bytes, void *stream);

/* ---- device plumbing for the ctypes layer and benchmarks ---- */
int lb_dev_malloc(void **ptr, size_t bytes);
int lb_dev_free(void *ptr);
int lb_memcpy_h2d(void *dst, const void *src, size_t bytes);
int lb_memcpy_d2h(void *dst, const void *src, size_t bytes);
int lb_memcpy_d2d(void *dst, const void *src, size_t bytes);
/* the same copies enqueued on `stream` (host memory may be pageable: the runtime
 * stages it, so the host buffer must stay valid until the stream is synchronised) */
int lb_memcpy_h2d_async(void *dst, const void *src, size_t bytes, void *stream);
int lb_memcpy_d2h_async(void *dst, const void *src, size_t bytes, void *stream);
int lb_memset_d(void *dst, int value, size_t bytes);
int lb_dev_synchronize(void);
int lb_stream_create(void **stream);
int lb_stream_destroy(void *stream);
int lb_stream_synchronize(void *stream);
int lb_event_create(void **event);
int lb_event_destroy(void *event);
int lb_event_record(void *event, void *stream);
int lb_event_synchronize(void *event);
int lb_event_elapsed_ms(void *start, void *stop, float *ms);
/* HIP graph capture of launch-bound loops: everything enqueued on `stream` between
 * begin and end becomes one graph, replayed by lb_graph_launch without per-kernel
 * host overhead. Entry points that allocate (lbd_gemm_w4a8 without a workspace
 * on first use) must not be captured. */
int lb_stream_begin_capture(void *stream);
int lb_stream_end_capture(void *stream, void **graph_exec);
int lb_graph_launch(void *graph_exec, void *stream);
int lb_graph_destroy(void *graph_exec);
/* plain streaming copy kernel of `bytes` (multiple of 16) on `stream`: the known-size
 * reference for scaling HBM traffic counters */
int lbd_copy_kernel(void *dst, const void *src, size_t bytes, void *stream);
/* plain streaming read of `bytes` (multiple of 16, below 4 GiB, 16-byte aligned) by
 * `workgroups` workgroups of `threads` (256 or 512) threads, `loads` (1, 2, 4 or 8)
 * 16-byte loads in flight per thread; each workgroup reads one contiguous range.
 * `sink` is one device dword (written only if the XOR of the data hits a fixed
 * value). The HBM read floor the decode GEMVs are measured against. */
int lbd_read_kernel(const void *src, size_t bytes, int workgroups, int threads, int loads, uint32_t *sink,
                    void *stream);
/* VALU issue-rate probe (no reference counterpart; the measurement behind the
 * instruction costs a kernel design relies on): form `op` (0 .. lbd_probe_forms() - 1,
 * in order v_fmac_f32, v_fma_f32, v_add_f32, v_mul_f32, v_and_b32, v_lshrrev_b32,
 * v_cvt_f32_ubyte1, v_cvt_f32_u32, v_bfe_u32, v_perm_b32, v_and_or_b32, v_fma_mix_f32,
 * v_dot4_i32_i8, v_pk_add_f16, v_cvt_scalef32_pk_f32_fp4), `iters` iterations of 32
 * instructions per thread (eight independent registers, four steps), `workgroups`
 * workgroups of 512 threads; `out`
 * receives workgroups * 512 floats of no meaning (they keep the work alive). */
int lbd_probe_valu(int op, int iters, int workgroups, float *out, void *stream);
int lbd_probe_forms(void);
/* Matrix-core / VALU sharing probe (no reference counterpart; the measurement behind
 * the int8 GEMM's arithmetic bound): per iteration 8 independent
 * v_mfma_i32_16x16x64_i8 (variant 0), 64 independent v_fmac_f32 (1), both with one
 * MFMA before each eight FMACs (2) or all MFMAs first (3); `workgroups` workgroups of
 * `threads` = 256 or 512 threads (one or two waves per SIMD at one workgroup per CU);
 * `out` receives workgroups * threads floats of no meaning. */
int lbd_probe_mfma_valu(int variant, int iters, int workgroups, int threads, float *out,
                        void *stream);
/* a kernel of `workgroups` x 512 threads that does nothing: the fixed cost of a launch */
int lbd_empty_kernel(int workgroups, void *stream);
/* Check of the one-row W4A8 quantizer's token scale (no reference counterpart: the
 * reference divides, src/lowbit/csrc/dispatch.c:231-257, and the paced GEMV replaces
 * that division by 127 with a multiply and two fused multiply-adds): on this device,
 * that replacement against the IEEE quotient a / 127.0f for every non-negative finite
 * float32 and +inf. out is two device dwords: out[0] = how many differ, out[1] = the
 * smallest differing bit pattern (0xFFFFFFFF when none). */
int lbd_probe_div127(uint32_t *out, void *stream);
/* Device-wide barrier probe (no reference counterpart; the measurement behind the
 * choice of one launch per decode phase over a persistent kernel): `rounds` (0 ..
 * 100000) barriers between `workgroups` (1 .. 1024) one-wave workgroups of one launch.
 * `mode` 0: one agent-scope atomic counter; 1: one flag per workgroup, polled by all;
 * 2: as 1 with agent-scope release / acquire fences around each barrier (what data
 * handed across it needs). `sync` is a device buffer of at least (64 + workgroups) * 4
 * bytes and `status` one device dword; both are cleared on `stream` before the launch
 * (so the call is not for graph capture). Every wait is bounded: status becomes 1 if
 * one timed out (a workgroup that was not resident), and the launch still ends. */
int lbd_probe_grid_barrier(int workgroups, int rounds, int mode, uint32_t *sync, size_t sync_bytes,
                           uint32_t *status, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* LOWBIT_HIP_H */
