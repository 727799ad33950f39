// C ABI of liblowbit_hip.so (declared in include/lowbit_hip.h).
//
// Replaces the reference's CPU driver (src/lowbit/csrc/dispatch.c): shape checks
// and return codes follow it (dispatch.c:160,205-208,279); the ISA dispatch and
// OpenMP tiling become a choice between two gfx950 regimes (VALU decode kernels
// for small M, matrix-core kernels otherwise), and the host-pointer entry points
// stage their operands through device memory owned by the calling thread.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>

#include "../../include/lowbit_hip.h"
#include "lb_internal.h"

namespace {

thread_local std::string t_error;
thread_local int t_status = 0;

int fail(int rc, const char *what) {
  t_error = what;
  t_status = rc;
  return rc;
}

int fail_hip(hipError_t e, const char *what) {
  t_error = std::string(what) + ": " + hipGetErrorString(e);
  t_status = LB_ERR_HIP;
  return LB_ERR_HIP;
}

int ok(int rc) {
  t_status = rc;
  return rc;
}

#define LB_HIP(call, what)                  \
  do {                                      \
    hipError_t e_ = (call);                 \
    if (e_ != hipSuccess) return fail_hip(e_, what); \
  } while (0)

inline size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

// ---------------------------------------------------------------- device info

struct DevInfo {
  int cus = 0;
  int lds = 0;
  bool gfx950 = false;
  char name[64] = {0};
};

std::mutex g_info_mu;
std::unordered_map<int, DevInfo> g_info;

int current_device(int *dev) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return fail(LB_ERR_UNAVAILABLE, "no HIP device");
  LB_HIP(hipGetDevice(dev), "hipGetDevice");
  return 0;
}

int device_info(DevInfo *out) {
  int dev = 0;
  int rc = current_device(&dev);
  if (rc < 0) return rc;
  std::lock_guard<std::mutex> lk(g_info_mu);
  auto it = g_info.find(dev);
  if (it == g_info.end()) {
    hipDeviceProp_t prop;
    LB_HIP(hipGetDeviceProperties(&prop, dev), "hipGetDeviceProperties");
    DevInfo d;
    d.cus = prop.multiProcessorCount;
    d.lds = (int)prop.sharedMemPerBlock;
    std::snprintf(d.name, sizeof d.name, "%s", prop.gcnArchName);
    d.gfx950 = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0;
    it = g_info.emplace(dev, d).first;
  }
  *out = it->second;
  return 0;
}

// ---------------------------------------------------------------- per-thread staging

// Device memory and a stream owned by one host thread on one device. Never freed:
// releasing HIP objects from thread-exit destructors can run after the runtime is
// gone, and the buffers are reused by every later call of the thread.
struct Ctx {
  hipStream_t stream = nullptr;
  char *buf = nullptr;
  size_t cap = 0;
  char *ws = nullptr;  // lbd_gemm_w4a8 workspace when the caller passes none
  size_t ws_cap = 0;
};

thread_local std::unordered_map<int, Ctx *> t_ctx;

int get_ctx(Ctx **out) {
  int dev = 0;
  int rc = current_device(&dev);
  if (rc < 0) return rc;
  auto it = t_ctx.find(dev);
  if (it == t_ctx.end()) {
    Ctx *c = new Ctx();
    hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
      delete c;
      return fail_hip(e, "hipStreamCreate");
    }
    it = t_ctx.emplace(dev, c).first;
  }
  *out = it->second;
  return 0;
}

int grow(char **buf, size_t *cap, size_t need, hipStream_t s) {
  if (need <= *cap) return 0;
  if (*buf) {
    LB_HIP(hipStreamSynchronize(s), "hipStreamSynchronize");
    LB_HIP(hipFree(*buf), "hipFree");
    *buf = nullptr;
    *cap = 0;
  }
  size_t sz = need < (size_t(1) << 20) ? (size_t(1) << 20) : need + need / 4;
  if (hipMalloc(reinterpret_cast<void **>(buf), sz) != hipSuccess) {
    *buf = nullptr;
    return fail(LB_ERR_ALLOC, "hipMalloc of staging memory failed");
  }
  *cap = sz;
  return 0;
}

// Carves 256-byte aligned pieces out of the thread's staging buffer.
struct Arena {
  size_t off = 0;
  size_t take(size_t n) {
    size_t o = off;
    off += align256(n);
    return o;
  }
};

// ---------------------------------------------------------------- validation

// Reference micro-tiles (src/lowbit/csrc/tiles.inc, kernels.py TILES): a Params that
// names any other (mr, nr) is rejected with -2, as the reference does.
bool tile_compiled(int mr, int nr) {
  static const int tiles[][2] = {{1, 1}, {1, 2}, {1, 4}, {2, 1}, {2, 2}, {2, 4},
                                 {4, 1}, {4, 2}, {4, 4}, {8, 1}, {8, 2}};
  for (auto &t : tiles)
    if (t[0] == mr && t[1] == nr) return true;
  return false;
}

int check_params(const lb_params *p, int M) {
  if (!p) return 0;
  int mr = p->mr > 0 ? p->mr : (M >= 4 ? 4 : 1);
  int nr = p->nr > 0 ? p->nr : 2;
  if (mr > 8) mr = 8;
  if (nr > 4) nr = 4;
  if (!tile_compiled(mr, nr)) return fail(LB_ERR_TILE, "lb_params names a micro-tile that does not exist");
  return 0;
}

int check_shape(int M, int Kp, int N, int block) {
  if (M <= 0 || N <= 0 || Kp <= 0 || Kp % block) return fail(LB_ERR_SHAPE, "bad shape (M, N, Kp <= 0 or Kp % block)");
  return 0;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// LOWBIT_ISA cap (read once): "gfx950" keeps GEMMs on the VALU kernels where the
// shape allows; anything else (or unset) leaves the choice automatic.
int env_cap() {
  static int cap = -2;
  if (cap == -2) {
    const char *e = std::getenv("LOWBIT_ISA");
    cap = (e && std::strcmp(e, "gfx950") == 0) ? LB_ISA_GFX950 : LB_ISA_GFX950_MFMA;
  }
  return cap;
}

// The regime a GEMM runs in. The request is first clamped to the LOWBIT_ISA cap
// (a matrix-core request under LOWBIT_ISA=gfx950 becomes a VALU request), as the
// reference clamps every request to its cap (src/lowbit/csrc/dispatch.c:77-80,151).
// A VALU request the shape cannot use then falls to the matrix-core kernels: they
// are the only ones that run it.
int choose_path(int fmt, int M, int Kp, const lb_params *p) {
  const bool valu_ok = lbk::gemv_eligible(fmt, M, Kp);
  int req = p ? p->isa : -1;
  if (req == LB_ISA_GFX950_MFMA && env_cap() < LB_ISA_GFX950_MFMA) req = env_cap();
  if (req == LB_ISA_GFX950_MFMA) return LB_ISA_GFX950_MFMA;
  return valu_ok ? LB_ISA_GFX950 : LB_ISA_GFX950_MFMA;
}

// ---------------------------------------------------------------- device-pointer cores

int run_w4a16(const lbk::GemmArgs &a, const lb_params *p, hipStream_t s) {
  int cus = 0;
  DevInfo di;
  if (device_info(&di) == 0) cus = di.cus;
  const int path = choose_path(lbk::F_W4A16, a.M, a.Kp, p);
  hipError_t e = path == LB_ISA_GFX950 ? lbk::launch_gemv(lbk::F_W4A16, a, cus, s)
                                       : lbk::launch_f32_mfma(lbk::F_W4A16, a, s);
  if (e != hipSuccess) return fail_hip(e, "W4A16 kernel launch");
  return ok(path);
}

int run_mxfp4(const lbk::GemmArgs &a, const lb_params *p, hipStream_t s) {
  int cus = 0;
  DevInfo di;
  if (device_info(&di) == 0) cus = di.cus;
  const int path = choose_path(lbk::F_MXFP4, a.M, a.Kp, p);
  hipError_t e = path == LB_ISA_GFX950 ? lbk::launch_gemv(lbk::F_MXFP4, a, cus, s)
                                       : lbk::launch_f32_mfma(lbk::F_MXFP4, a, s);
  if (e != hipSuccess) return fail_hip(e, "MXFP4 kernel launch");
  return ok(path);
}

size_t w4a8_ws_bytes(int M, int Kp) {
  return align256(lbk::tiled_xq_bytes(M, Kp)) + align256((size_t)M * 4) + align256(lbk::tiled_asum_bytes(M, Kp));
}

// The caller's workspace of `need` bytes (checked) or, when it passed none, the
// per-thread buffer.
int take_workspace(size_t need, size_t given_bytes, hipStream_t s, char **ws) {
  if (*ws) {
    if (given_bytes < need) return fail(LB_ERR_ARG, "workspace too small");
    if ((reinterpret_cast<uintptr_t>(*ws) & 255) != 0) return fail(LB_ERR_ARG, "workspace must be 256-byte aligned");
    return 0;
  }
  Ctx *c = nullptr;
  int rc = get_ctx(&c);
  if (rc < 0) return rc;
  if ((rc = grow(&c->ws, &c->ws_cap, need, s)) < 0) return rc;
  *ws = c->ws;
  return 0;
}

int w4a8_workspace(int M, int Kp, size_t given_bytes, hipStream_t s, char **ws) {
  return take_workspace(w4a8_ws_bytes(M, Kp), given_bytes, s, ws);
}

// bf16x3 GEMM on t16 (or, f8, t16f8) weights: split the activations into `ws`,
// then the GEMM.
int run_bf3(int fmt, const lbk::GemmArgs &a0, char *ws, hipStream_t s, bool f8 = false) {
  int cus = 0;
  DevInfo di;
  if (device_info(&di) == 0) cus = di.cus;
  lbk::GemmArgs a = a0;
  a.x3 = reinterpret_cast<const uint4 *>(ws);
  hipError_t e;
  if (fmt == lbk::F_W4A16) {
    // two float16 terms per row and its exponent (within the bf16x3 workspace)
    int *xexp = reinterpret_cast<int *>(ws + lbk::x2h_exp_offset(a.M, a.Kp));
    a.xexp = xexp;
    e = lbk::launch_split2h(a.x, a.M, a.Kp, reinterpret_cast<uint4 *>(ws), xexp, s);
  } else {
    e = lbk::launch_split3(fmt, a.x, a.M, a.Kp, reinterpret_cast<uint4 *>(ws), s);
  }
  if (e != hipSuccess) return fail_hip(e, "activation split launch");
  e = lbk::launch_bf3_gemm(fmt, a, cus, s, f8);
  if (e != hipSuccess) return fail_hip(e, "bf16x3 GEMM launch");
  return ok(LB_ISA_GFX950_MFMA);
}

// The workspace of a bf16x3 call: the split activations, then (K split over the
// workgroups, where the shape takes it) the slices' partial outputs. A caller's
// workspace of at least lbd_bf16x3_workspace_bytes bytes runs the unsplit GEMM; one
// of lbd_bf16x3_workspace_bytes_split bytes, or none (the per-thread buffer), the
// split one. The two give results within the same bound, not the same bits.
int bf3_call(int fmt, lbk::GemmArgs &a, char *ws, size_t given, hipStream_t s, bool f8 = false) {
  const size_t x3 = align256(lbk::x3_bytes(a.M, a.Kp)), part = lbk::bf3_part_bytes(fmt, a.M, a.N, a.Kp);
  const bool own = ws == nullptr;
  const int rc = take_workspace(own ? x3 + part : lbk::x3_bytes(a.M, a.Kp), given, s, &ws);
  if (rc < 0) return rc;
  if (part && (own || given >= x3 + part)) a.ypart = reinterpret_cast<float *>(ws + x3);
  return run_bf3(fmt, a, ws, s, f8);
}

// Shared checks of the t16 GEMM entry points (32-bit offsets inside the kernels).
int check_t16(int M, int Kp, int N, bool f8 = false) {
  if ((size_t)M * Kp * 4 > 0xFFFFFFF0u || lbk::x3_bytes(M, Kp) > 0xFFFFFFF0u)
    return fail(LB_ERR_SHAPE, "activations above 4 GiB");
  if ((f8 ? lbk::t16f8_qw_bytes(N, Kp) : lbk::t16_qw_bytes(N, Kp)) > 0xFFFFFFF0u)
    return fail(LB_ERR_SHAPE, "t16 weights above 4 GiB");
  return 0;
}

// Whether a host-pointer call can take the t16 matrix-core route (the limits check_t16
// enforces, tested without recording an error).
bool host_t16_fits(int M, int Kp, int N) {
  return (size_t)M * Kp * 4 <= 0xFFFFFFF0u && lbk::x3_bytes(M, Kp) <= 0xFFFFFFF0u &&
         lbk::t16_qw_bytes(N, Kp) <= 0xFFFFFFF0u;
}

// fp32 activations in; quantized inside (fused into the GEMV, or a quantizer
// kernel into `ws` before the MFMA kernel).
int run_w4a8(const lbk::GemmArgs &a, const lb_params *p, char *ws, hipStream_t s) {
  int cus = 0;
  DevInfo di;
  if (device_info(&di) == 0) cus = di.cus;
  // t16 weights exist only for the matrix-core kernel
  const int path = a.wt16 ? LB_ISA_GFX950_MFMA : choose_path(lbk::F_W4A8, a.M, a.Kp, p);
  if (path == LB_ISA_GFX950) {
    hipError_t e = lbk::launch_gemv(lbk::F_W4A8, a, cus, s);
    if (e != hipSuccess) return fail_hip(e, "W4A8 GEMV launch");
    return ok(path);
  }
  lbk::GemmArgs q = a;
  // quantized activations in the tiled layout the MFMA kernel reads
  const size_t xq_bytes = align256(lbk::tiled_xq_bytes(a.M, a.Kp));
  int8_t *xq = reinterpret_cast<int8_t *>(ws);
  float *xs = reinterpret_cast<float *>(ws + xq_bytes);
  int32_t *asum = reinterpret_cast<int32_t *>(ws + xq_bytes + align256((size_t)a.M * 4));
  hipError_t e = lbk::launch_quant(a.x, a.M, a.Kp, xq, xs, asum, true, s);
  if (e != hipSuccess) return fail_hip(e, "quantizer launch");
  q.xq = xq;
  q.xs = xs;
  q.asum = asum;
  q.tiled = true;
  e = lbk::launch_w4a8_mfma(q, nullptr, cus, s);
  if (e != hipSuccess) return fail_hip(e, "W4A8 MFMA launch");
  return ok(path);
}

int run_w4a8_q(const lbk::GemmArgs &a, const lb_params *p, hipStream_t s) {
  int cus = 0;
  DevInfo di;
  if (device_info(&di) == 0) cus = di.cus;
  const int path = choose_path(lbk::F_W4A8Q, a.M, a.Kp, p);
  hipError_t e = path == LB_ISA_GFX950 ? lbk::launch_gemv(lbk::F_W4A8Q, a, cus, s)
                                       : lbk::launch_w4a8_mfma(a, nullptr, cus, s);
  if (e != hipSuccess) return fail_hip(e, "W4A8 kernel launch");
  return ok(path);
}

int run_group_acc(const int8_t *xq, const int32_t *asum, int M, int Kp, const uint8_t *qw,
                  const uint8_t *zeros, int N, int32_t *out, int isa, hipStream_t s) {
  hipError_t e;
  int path;
  if (isa == LB_ISA_GFX950_MFMA) {
    lbk::GemmArgs a;
    a.xq = xq;
    a.asum = asum;
    a.qw = qw;
    a.zeros = zeros;
    a.M = M;
    a.Kp = Kp;
    a.N = N;
    int cus = 0;
    DevInfo di;
    if (device_info(&di) == 0) cus = di.cus;
    e = lbk::launch_w4a8_mfma(a, out, cus, s);
    path = LB_ISA_GFX950_MFMA;
  } else {
    e = lbk::launch_groupacc_dot4(xq, asum, M, Kp, qw, zeros, N, out, s);
    path = LB_ISA_GFX950;
  }
  if (e != hipSuccess) return fail_hip(e, "group accumulator launch");
  return ok(path);
}

}  // namespace

// ====================================================================== C ABI

extern "C" {

int lb_version(void) { return 1; }

int lb_cpu_isa(void) {
  DevInfo d;
  if (device_info(&d) < 0) return LB_ERR_UNAVAILABLE;
  return d.gfx950 ? LB_ISA_GFX950_MFMA : LB_ERR_UNAVAILABLE;
}

int lb_active_isa(void) {
  const int top = lb_cpu_isa();
  if (top < 0) return top;
  return env_cap() < top ? env_cap() : top;
}

int lb_has_vnni(void) { return 0; }
int lb_has_openmp(void) { return 0; }
int lb_max_threads(void) { return 1; }

int lb_effective_isa(int kind, int requested) {
  (void)kind;
  const int top = lb_active_isa();
  if (top < 0) return top;
  if (requested == LB_ISA_GFX950) return LB_ISA_GFX950;
  return top;
}

int lb_device_info(char *name, int name_len, int *compute_units, int *lds_bytes) {
  DevInfo d;
  int rc = device_info(&d);
  if (rc < 0) return rc;
  if (name && name_len > 0) std::snprintf(name, (size_t)name_len, "%s", d.name);
  if (compute_units) *compute_units = d.cus;
  if (lds_bytes) *lds_bytes = d.lds;
  return ok(0);
}

const char *lb_last_error(void) { return t_error.c_str(); }
int lb_last_status(void) { return t_status; }

// ---------------------------------------------------------------- device-pointer GEMMs

int lbd_gemm_w4a16(const float *x, int M, int Kp, const uint8_t *qw, const float *scales,
                   const uint8_t *zeros, int N, float *y, const lb_params *p, void *stream) {
  int rc = check_shape(M, Kp, N, LB_GROUP);
  if (rc < 0) return rc;
  if ((rc = check_params(p, M)) < 0) return rc;
  if (!x || !qw || !scales || !y) return fail(LB_ERR_ARG, "null pointer");
  if (!aligned16(x) || !aligned16(qw)) return fail(LB_ERR_ARG, "x and qw must be 16-byte aligned");
  lbk::GemmArgs a;
  a.x = x; a.qw = qw; a.scales = scales; a.zeros = zeros; a.y = y;
  a.M = M; a.Kp = Kp; a.N = N;
  return run_w4a16(a, p, static_cast<hipStream_t>(stream));
}

int lbd_gemm_mxfp4(const float *x, int M, int Kp, const uint8_t *qw, const uint8_t *e8m0,
                   int N, float *y, const lb_params *p, void *stream) {
  int rc = check_shape(M, Kp, N, LB_MXBLOCK);
  if (rc < 0) return rc;
  if ((rc = check_params(p, M)) < 0) return rc;
  if (!x || !qw || !e8m0 || !y) return fail(LB_ERR_ARG, "null pointer");
  if (!aligned16(x) || !aligned16(qw)) return fail(LB_ERR_ARG, "x and qw must be 16-byte aligned");
  lbk::GemmArgs a;
  a.x = x; a.qw = qw; a.e8m0 = e8m0; a.y = y;
  a.M = M; a.Kp = Kp; a.N = N;
  return run_mxfp4(a, p, static_cast<hipStream_t>(stream));
}

size_t lbd_w4a8_workspace_bytes(int M, int Kp) {
  if (M <= 0 || Kp <= 0) return 0;
  return w4a8_ws_bytes(M, Kp);
}

int lbd_gemm_w4a8(const float *x, int M, int Kp, const uint8_t *qw, const float *scales,
                  const uint8_t *zeros, int N, float *y, const lb_params *p, void *workspace,
                  size_t workspace_bytes, void *stream) {
  int rc = check_shape(M, Kp, N, LB_GROUP);
  if (rc < 0) return rc;
  if ((rc = check_params(p, M)) < 0) return rc;
  if (!x || !qw || !scales || !y) return fail(LB_ERR_ARG, "null pointer");
  if (!aligned16(x) || !aligned16(qw)) return fail(LB_ERR_ARG, "x and qw must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  lbk::GemmArgs a;
  a.x = x; a.qw = qw; a.scales = scales; a.zeros = zeros; a.y = y;
  a.M = M; a.Kp = Kp; a.N = N;
  char *ws = static_cast<char *>(workspace);
  if (choose_path(lbk::F_W4A8, M, Kp, p) == LB_ISA_GFX950_MFMA &&
      (rc = w4a8_workspace(M, Kp, workspace_bytes, s, &ws)) < 0)
    return rc;
  return run_w4a8(a, p, ws, s);
}

int lbd_gemm_path(int kind, int M, int Kp, const lb_params *p) {
  static const int fmts[] = {lbk::F_W4A16, lbk::F_MXFP4, lbk::F_W4A8};
  if (kind < 0 || kind > 2) return fail(LB_ERR_ARG, "unknown GEMM kind");
  if (M <= 0 || Kp <= 0) return fail(LB_ERR_SHAPE, "bad shape");
  const int rc = check_params(p, M);
  if (rc < 0) return rc;
  return ok(choose_path(fmts[kind], M, Kp, p));
}

int lbd_gemm_plan(int kind, int M, int N, int Kp, const lb_params *p, lbd_plan *out) {
  static const int fmts[] = {lbk::F_W4A16, lbk::F_MXFP4, lbk::F_W4A8};
  if (kind < 0 || kind > 2 || !out) return fail(LB_ERR_ARG, "unknown GEMM kind or null plan");
  int rc = check_shape(M, Kp, N, kind == 1 ? LB_MXBLOCK : LB_GROUP);
  if (rc < 0) return rc;
  std::memset(out, 0, sizeof *out);
  out->path = choose_path(fmts[kind], M, Kp, p);
  if (out->path != LB_ISA_GFX950) return ok(out->path);
  int cus = 0;
  DevInfo di;
  if (device_info(&di) == 0) cus = di.cus;
  lbk::GemmArgs a;
  a.M = M; a.Kp = Kp; a.N = N;
  lbk::GemvPlan g;
  hipError_t e = lbk::launch_gemv(fmts[kind], a, cus, nullptr, &g);
  if (e != hipSuccess) return fail_hip(e, "small-M plan");
  out->workgroups = g.workgroups;
  out->rows_per_wave = g.rows_per_wave;
  out->rows_held = g.rows_held;
  out->chunks_per_lane = g.chunks_per_lane;
  out->two_rows_per_load = g.two_rows_per_load;
  out->act_rows = g.act_rows;
  out->k_slices = g.k_slices;
  return ok(out->path);
}

int lbd_quantize_int4(const float *w, int N, int K, int asym, int signed_max, uint8_t *qw, float *scales,
                      uint8_t *zeros, void *stream) {
  if (N <= 0 || K <= 0) return fail(LB_ERR_SHAPE, "bad shape");
  if (asym && signed_max) return fail(LB_ERR_ARG, "signed-max is a symmetric rule");
  if (!w || !qw || !scales || (asym && !zeros)) return fail(LB_ERR_ARG, "null pointer");
  const int mode = asym ? 2 : (signed_max ? 1 : 0);
  hipError_t e = lbk::launch_quantize_int4(w, N, K, mode, LB_GROUP, qw, scales, zeros,
                                           static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail_hip(e, "int4 quantizer launch");
  return ok(0);
}

int lbd_quantize_int4_g32(const float *w, int N, int K, int asym, int signed_max, uint8_t *qw, float *scales,
                          uint8_t *zeros, void *stream) {
  if (N <= 0 || K <= 0) return fail(LB_ERR_SHAPE, "bad shape");
  if (asym && signed_max) return fail(LB_ERR_ARG, "signed-max is a symmetric rule");
  if (!w || !qw || !scales || (asym && !zeros)) return fail(LB_ERR_ARG, "null pointer");
  const int mode = asym ? 2 : (signed_max ? 1 : 0);
  hipError_t e = lbk::launch_quantize_int4(w, N, K, mode, LB_G32, qw, scales, zeros,
                                           static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail_hip(e, "int4 g32 quantizer launch");
  return ok(0);
}

int lbd_quantize_mxfp4(const float *w, int N, int K, uint8_t *qw, uint8_t *e8m0, void *stream) {
  if (N <= 0 || K <= 0) return fail(LB_ERR_SHAPE, "bad shape");
  if (!w || !qw || !e8m0) return fail(LB_ERR_ARG, "null pointer");
  hipError_t e = lbk::launch_quantize_mxfp4(w, N, K, qw, e8m0, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail_hip(e, "MXFP4 quantizer launch");
  return ok(0);
}

int lbd_int4_t16_bytes(int N, int Kp, size_t *qwt_bytes, size_t *st_bytes, size_t *zt_bytes) {
  int rc = check_shape(1, Kp, N, LB_GROUP);
  if (rc < 0) return rc;
  if (qwt_bytes) *qwt_bytes = lbk::t16_qw_bytes(N, Kp);
  if (st_bytes) *st_bytes = lbk::t16_group_entries(N, Kp) * 4;
  if (zt_bytes) *zt_bytes = lbk::t16_group_entries(N, Kp);
  return ok(0);
}

int lbd_repack_int4_t16(const uint8_t *qw, const float *scales, const uint8_t *zeros, int N, int Kp,
                        uint8_t *qwt, float *st, uint8_t *zt, void *stream) {
  int rc = check_shape(1, Kp, N, LB_GROUP);
  if (rc < 0) return rc;
  if (!qw || !scales || !qwt || !st || (zeros && !zt)) return fail(LB_ERR_ARG, "null pointer");
  if (!aligned16(qw) || !aligned16(qwt)) return fail(LB_ERR_ARG, "qw and qwt must be 16-byte aligned");
  if (lbk::t16_qw_bytes(N, Kp) > 0xFFFFFFF0u) return fail(LB_ERR_SHAPE, "t16 weights above 4 GiB");
  hipError_t e = lbk::launch_repack_int4_t16(qw, scales, zeros, N, Kp, qwt, st, zeros ? zt : nullptr,
                                             static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail_hip(e, "t16 repack launch");
  return ok(0);
}

size_t lbd_bf16x3_workspace_bytes(int M, int Kp) {
  if (M <= 0 || Kp <= 0) return 0;
  return lbk::x3_bytes(M, Kp);
}

size_t lbd_bf16x3_workspace_bytes_split(int kind, int M, int N, int Kp) {
  if (M <= 0 || N <= 0 || Kp <= 0 || (kind != 0 && kind != 1)) return 0;
  return align256(lbk::x3_bytes(M, Kp)) + lbk::bf3_part_bytes(kind == 1 ? lbk::F_MXFP4 : lbk::F_W4A16, M, N, Kp);
}

int lbd_gemm_w4a16_t16(const float *x, int M, int Kp, const uint8_t *qwt, const float *st, const uint8_t *zt,
                       int N, float *y, const lb_params *p, void *workspace, size_t workspace_bytes,
                       void *stream) {
  int rc = check_shape(M, Kp, N, LB_GROUP);
  if (rc < 0) return rc;
  if ((rc = check_params(p, M)) < 0) return rc;
  if (!x || !qwt || !st || !y) return fail(LB_ERR_ARG, "null pointer");
  if (!aligned16(x) || !aligned16(qwt)) return fail(LB_ERR_ARG, "x and qwt must be 16-byte aligned");
  if ((rc = check_t16(M, Kp, N)) < 0) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  lbk::GemmArgs a;
  a.x = x; a.qw = qwt; a.scales = st; a.zeros = zt; a.y = y;
  a.M = M; a.Kp = Kp; a.N = N;
  a.wt16 = true;
  char *ws = static_cast<char *>(workspace);
  return bf3_call(lbk::F_W4A16, a, ws, workspace_bytes, s);
}

int lbd_int4_t16f8_bytes(int N, int Kp, size_t *qwt8_bytes, size_t *st_bytes) {
  int rc = check_shape(1, Kp, N, LB_GROUP);
  if (rc < 0) return rc;
  if (qwt8_bytes) *qwt8_bytes = lbk::t16f8_qw_bytes(N, Kp);
  if (st_bytes) *st_bytes = lbk::t16_group_entries(N, Kp) * 4;
  return ok(0);
}

int lbd_repack_int4_t16f8(const uint8_t *qw, const float *scales, const uint8_t *zeros, int N, int Kp,
                          uint8_t *qwt8, float *st, void *stream) {
  int rc = check_shape(1, Kp, N, LB_GROUP);
  if (rc < 0) return rc;
  if (!qw || !scales || !qwt8 || !st) return fail(LB_ERR_ARG, "null pointer");
  if (!aligned16(qw) || !aligned16(qwt8)) return fail(LB_ERR_ARG, "qw and qwt8 must be 16-byte aligned");
  if (lbk::t16f8_qw_bytes(N, Kp) > 0xFFFFFFF0u) return fail(LB_ERR_SHAPE, "t16f8 weights above 4 GiB");
  hipError_t e = lbk::launch_repack_int4_t16f8(qw, scales, zeros, N, Kp, qwt8, st, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail_hip(e, "t16f8 repack launch");
  return ok(0);
}

int lbd_w4a16_prefers_t16f8(int M, int N, int Kp) {
  int rc = check_shape(M, Kp, N, LB_GROUP);
  if (rc < 0) return rc;
  int cus = 0;
  DevInfo di;
  if (device_info(&di) == 0) cus = di.cus;
  return lbk::w4a16_prefers_t16f8(M, N, Kp, cus) ? 1 : 0;
}

int lbd_gemm_w4a16_t16f8(const float *x, int M, int Kp, const uint8_t *qwt8, const float *st, int N, float *y,
                         const lb_params *p, void *workspace, size_t workspace_bytes, void *stream) {
  int rc = check_shape(M, Kp, N, LB_GROUP);
  if (rc < 0) return rc;
  if ((rc = check_params(p, M)) < 0) return rc;
  if (!x || !qwt8 || !st || !y) return fail(LB_ERR_ARG, "null pointer");
  if (!aligned16(x) || !aligned16(qwt8)) return fail(LB_ERR_ARG, "x and qwt8 must be 16-byte aligned");
  if ((rc = check_t16(M, Kp, N, true)) < 0) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  lbk::GemmArgs a;
  a.x = x; a.qw = qwt8; a.scales = st; a.y = y;
  a.M = M; a.Kp = Kp; a.N = N;
  a.wt16 = true;
  char *ws = static_cast<char *>(workspace);
  return bf3_call(lbk::F_W4A16, a, ws, workspace_bytes, s, true);
}

int lbd_mxfp4_t16_bytes(int N, int Kp, size_t *qwt_bytes, size_t *et_bytes) {
  int rc = check_shape(1, Kp, N, LB_MXBLOCK);
  if (rc < 0) return rc;
  if (qwt_bytes) *qwt_bytes = lbk::t16_qw_bytes(N, Kp);
  if (et_bytes) *et_bytes = lbk::t16_e8m0_bytes(N, Kp);
  return ok(0);
}

int lbd_repack_mxfp4_t16(const uint8_t *qw, const uint8_t *e8m0, int N, int Kp, uint8_t *qwt, uint8_t *et,
                         void *stream) {
  int rc = check_shape(1, Kp, N, LB_MXBLOCK);
  if (rc < 0) return rc;
  if (!qw || !e8m0 || !qwt || !et) return fail(LB_ERR_ARG, "null pointer");
  if (!aligned16(qw) || !aligned16(qwt)) return fail(LB_ERR_ARG, "qw and qwt must be 16-byte aligned");
  if (lbk::t16_qw_bytes(N, Kp) > 0xFFFFFFF0u) return fail(LB_ERR_SHAPE, "t16 weights above 4 GiB");
  hipError_t e = lbk::launch_repack_mxfp4_t16(qw, e8m0, N, Kp, qwt, et, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail_hip(e, "t16 repack launch");
  return ok(0);
}

int lbd_gemm_mxfp4_t16(const float *x, int M, int Kp, const uint8_t *qwt, const uint8_t *et, int N, float *y,
                       const lb_params *p, void *workspace, size_t workspace_bytes, void *stream) {
  int rc = check_shape(M, Kp, N, LB_MXBLOCK);
  if (rc < 0) return rc;
  if ((rc = check_params(p, M)) < 0) return rc;
  if (!x || !qwt || !et || !y) return fail(LB_ERR_ARG, "null pointer");
  if (!aligned16(x) || !aligned16(qwt)) return fail(LB_ERR_ARG, "x and qwt must be 16-byte aligned");
  if ((rc = check_t16(M, Kp, N)) < 0) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  lbk::GemmArgs a;
  a.x = x; a.qw = qwt; a.e8m0 = et; a.y = y;
  a.M = M; a.Kp = Kp; a.N = N;
  a.wt16 = true;
  char *ws = static_cast<char *>(workspace);
  return bf3_call(lbk::F_MXFP4, a, ws, workspace_bytes, s);
}

}  // extern "C"

namespace {

int check_w4a8_t16(const float *x, int M, int Kp, const uint8_t *qwt, const float *st, const uint8_t *zt, int N,
                   float *y, const lb_params *p) {
  int rc = check_shape(M, Kp, N, LB_GROUP);
  if (rc < 0) return rc;
  if ((rc = check_params(p, M)) < 0) return rc;
  if (!x || !qwt || !st || !y) return fail(LB_ERR_ARG, "null pointer");
  if (!aligned16(x) || !aligned16(qwt) || !aligned16(st))
    return fail(LB_ERR_ARG, "x, qwt and st must be 16-byte aligned");
  if (zt && (reinterpret_cast<uintptr_t>(zt) & 3)) return fail(LB_ERR_ARG, "zt must be 4-byte aligned");
  if (lbk::t16_qw_bytes(N, Kp) > 0xFFFFFFF0u) return fail(LB_ERR_SHAPE, "t16 weights above 4 GiB");
  return 0;
}

lbk::GemmArgs w4a8_t16_args(const float *x, int M, int Kp, const uint8_t *qwt, const float *st, const uint8_t *zt,
                            int N, float *y) {
  lbk::GemmArgs a;
  a.x = x; a.qw = qwt; a.scales = st; a.zeros = zt; a.y = y;
  a.M = M; a.Kp = Kp; a.N = N;
  a.wt16 = true;
  return a;
}

}  // namespace

extern "C" {

int lbd_gemm_w4a8_t16(const float *x, int M, int Kp, const uint8_t *qwt, const float *st, const uint8_t *zt,
                      int N, float *y, const lb_params *p, void *workspace, size_t workspace_bytes,
                      void *stream) {
  int rc = check_w4a8_t16(x, M, Kp, qwt, st, zt, N, y, p);
  if (rc < 0) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  char *ws = static_cast<char *>(workspace);
  if ((rc = w4a8_workspace(M, Kp, workspace_bytes, s, &ws)) < 0) return rc;
  return run_w4a8(w4a8_t16_args(x, M, Kp, qwt, st, zt, N, y), p, ws, s);
}

int lbd_gemm_w4a8_q(const int8_t *xq, const float *xs, const int32_t *asum, int M, int Kp,
                    const uint8_t *qw, const float *scales, const uint8_t *zeros, int N, float *y,
                    const lb_params *p, void *stream) {
  int rc = check_shape(M, Kp, N, LB_GROUP);
  if (rc < 0) return rc;
  if ((rc = check_params(p, M)) < 0) return rc;
  if (!xq || !xs || !asum || !qw || !scales || !y) return fail(LB_ERR_ARG, "null pointer");
  if (!aligned16(xq) || !aligned16(qw)) return fail(LB_ERR_ARG, "xq and qw must be 16-byte aligned");
  lbk::GemmArgs a;
  a.xq = xq; a.xs = xs; a.asum = asum; a.qw = qw; a.scales = scales; a.zeros = zeros; a.y = y;
  a.M = M; a.Kp = Kp; a.N = N;
  return run_w4a8_q(a, p, static_cast<hipStream_t>(stream));
}

int lbd_quant_act_int8(const float *x, int M, int Kp, int8_t *xq, float *xs, int32_t *asum,
                       void *stream) {
  if (M <= 0 || Kp <= 0 || Kp % LB_GROUP) return fail(LB_ERR_SHAPE, "bad shape");
  if (!x || !xq || !xs || !asum) return fail(LB_ERR_ARG, "null pointer");
  if (!aligned16(x) || !aligned16(xq)) return fail(LB_ERR_ARG, "x and xq must be 16-byte aligned");
  hipError_t e = lbk::launch_quant(x, M, Kp, xq, xs, asum, false, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail_hip(e, "quantizer launch");
  return ok(0);
}

int lbd_w4a8_group_acc(const int8_t *xq, const int32_t *asum, int M, int Kp, const uint8_t *qw,
                       const uint8_t *zeros, int N, int32_t *out, int isa, void *stream) {
  int rc = check_shape(M, Kp, N, LB_GROUP);
  if (rc < 0) return rc;
  if (!xq || !asum || !qw || !out) return fail(LB_ERR_ARG, "null pointer");
  if (!aligned16(xq) || !aligned16(qw)) return fail(LB_ERR_ARG, "xq and qw must be 16-byte aligned");
  return run_group_acc(xq, asum, M, Kp, qw, zeros, N, out, isa, static_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------- decoder-layer operations

#define LB_LAUNCH(call, what)                    \
  do {                                           \
    hipError_t e_ = (call);                      \
    if (e_ != hipSuccess) return fail_hip(e_, what); \
    return ok(0);                                \
  } while (0)

int lbd_embed(const float *table, int vocab, int hidden, const int32_t *tok, int T, float *x, void *stream) {
  if (vocab <= 0 || hidden <= 0 || T <= 0) return fail(LB_ERR_SHAPE, "bad shape");
  if (!table || !tok || !x) return fail(LB_ERR_ARG, "null pointer");
  LB_LAUNCH(lbk::launch_embed(table, vocab, hidden, tok, T, x, static_cast<hipStream_t>(stream)), "embed launch");
}

int lbd_rmsnorm(const float *x, const float *w, int T, int hidden, float eps, float *y, void *stream) {
  if (T <= 0 || hidden <= 0) return fail(LB_ERR_SHAPE, "bad shape");
  if (!x || !w || !y) return fail(LB_ERR_ARG, "null pointer");
  LB_LAUNCH(lbk::launch_rmsnorm(x, w, T, hidden, eps, y, static_cast<hipStream_t>(stream)), "rmsnorm launch");
}

int lbd_qkv_rope(float *qkv, const float *bias, int T, int H, int KV, int D, const float *cos_table,
                 const float *sin_table, const int32_t *pos, int max_pos, float *k_cache, float *v_cache, int cap,
                 void *stream) {
  if (T <= 0 || H <= 0 || KV <= 0 || H % KV || (D != 32 && D != 64 && D != 128) || max_pos <= 0 || cap <= 0)
    return fail(LB_ERR_SHAPE, "bad shape");
  if (!qkv || !cos_table || !sin_table || !pos || !k_cache || !v_cache) return fail(LB_ERR_ARG, "null pointer");
  LB_LAUNCH(lbk::launch_qkv_rope(qkv, bias, T, H, KV, D, cos_table, sin_table, pos, max_pos, k_cache, v_cache, cap,
                                 static_cast<hipStream_t>(stream)),
            "qkv rope launch");
}

int lbd_attention(const float *q, int qstride, const float *k_cache, const float *v_cache, int T, int H, int KV, int D,
                  const int32_t *pos, int cap, float *out, void *stream) {
  if (T <= 0 || H <= 0 || KV <= 0 || H % KV || (D != 32 && D != 64 && D != 128) || cap <= 0 || cap > 16000 ||
      qstride < H * D)
    return fail(LB_ERR_SHAPE, "bad shape");
  if (!q || !k_cache || !v_cache || !pos || !out) return fail(LB_ERR_ARG, "null pointer");
  if ((reinterpret_cast<uintptr_t>(k_cache) & 15) != 0) return fail(LB_ERR_ARG, "k_cache must be 16-byte aligned");
  LB_LAUNCH(lbk::launch_attention(q, qstride, k_cache, v_cache, T, H, KV, D, pos, cap, out,
                                  static_cast<hipStream_t>(stream)),
            "attention launch");
}

int lbd_swiglu(const float *gu, int T, int I, float *out, void *stream) {
  if (T <= 0 || I <= 0) return fail(LB_ERR_SHAPE, "bad shape");
  if (!gu || !out) return fail(LB_ERR_ARG, "null pointer");
  LB_LAUNCH(lbk::launch_swiglu(gu, T, I, out, static_cast<hipStream_t>(stream)), "swiglu launch");
}

int lbd_swiglu_pairs(const float *gu, int T, int I, float *out, void *stream) {
  if (T <= 0 || I <= 0) return fail(LB_ERR_SHAPE, "bad shape");
  if (!gu || !out) return fail(LB_ERR_ARG, "null pointer");
  if ((reinterpret_cast<uintptr_t>(gu) & 7) != 0) return fail(LB_ERR_ARG, "gu must be 8-byte aligned");
  LB_LAUNCH(lbk::launch_swiglu_pairs(gu, T, I, out, static_cast<hipStream_t>(stream)), "swiglu launch");
}

int lbd_add(float *x, const float *y, size_t n, void *stream) {
  if (!x || !y) return fail(LB_ERR_ARG, "null pointer");
  if (n == 0) return ok(0);
  LB_LAUNCH(lbk::launch_add(x, y, n, static_cast<hipStream_t>(stream)), "add launch");
}

int lbd_argmax(const float *v, int n, int32_t *tok, int32_t *pos, int inc, int32_t *hist, int hist_len, void *stream) {
  if (n <= 0) return fail(LB_ERR_SHAPE, "bad shape");
  if (!v || !tok) return fail(LB_ERR_ARG, "null pointer");
  LB_LAUNCH(lbk::launch_argmax(v, n, tok, pos, inc, hist, hist_len, static_cast<hipStream_t>(stream)),
            "argmax launch");
}

// ---------------------------------------------------------------- fused decode GEMVs

}  // extern "C"

namespace {

static_assert(LBD_ARGMAX_SLOTS == lbk::kArgmaxSlots, "argmax slot count of the ABI and the kernels");

// Checks shared by the fused GEMVs; fills the fusion fields of `a`.
int fused_args(int fmt, const lbd_fusion *f, lbk::GemmArgs &a) {
  if (!lbk::gemv_eligible(fmt, a.M, a.Kp))
    return fail(LB_ERR_SHAPE, "fused GEMVs take the small-M kernels only (M <= 4, Kp within their limit)");
  if (!f) return 0;
  if (f->norm_w && f->swiglu) return fail(LB_ERR_ARG, "RMSNorm and SwiGLU prologues are exclusive");
  if ((f->norm_w || f->swiglu || f->argmax_key) && a.M != 1)
    return fail(LB_ERR_ARG, "prologues and the argmax key need M == 1");
  if (f->norm_w && !aligned16(f->norm_w)) return fail(LB_ERR_ARG, "norm_w must be 16-byte aligned");
  if (f->argmax_key && (reinterpret_cast<uintptr_t>(f->argmax_key) & 7) != 0)
    return fail(LB_ERR_ARG, "argmax_key must be 8-byte aligned");
  if (f->glu && (f->residual || f->argmax_key))
    return fail(LB_ERR_ARG, "the glu epilogue excludes the residual and the argmax key");
  if (f->glu && (a.N & 1)) return fail(LB_ERR_SHAPE, "the glu epilogue takes an even N (gate/up row pairs)");
  if (f->attn_part) {
    const int D = f->attn_head_dim;
    if (a.M != 1 || f->norm_w || f->swiglu)
      return fail(LB_ERR_ARG, "the attention-merge prologue needs M == 1 and no other prologue");
    if ((D != 32 && D != 64 && D != 128) || a.Kp % D || a.Kp > 2048 || f->attn_cap <= 0 ||
        f->attn_cap > 16000 || lbk::attn_slices(D, f->attn_cap) > lbk::kAttnMaxFusedSlices)
      return fail(LB_ERR_SHAPE, "attention merge: Kp = heads x head_dim <= 2048, at most 8 key slices");
    if (!aligned16(f->attn_part)) return fail(LB_ERR_ARG, "attn_part must be 16-byte aligned");
    a.attn_part = f->attn_part;
    a.attn_ns = lbk::attn_slices(D, f->attn_cap);
    a.attn_d = D;
  }
  a.norm_w = f->norm_w;
  a.norm_eps = f->norm_eps;
  a.swiglu = f->swiglu != 0;
  a.bias = f->bias;
  a.res = f->residual;
  a.amax_key = f->argmax_key;
  a.glu = f->glu != 0;
  return 0;
}

int run_fused(int fmt, const lbk::GemmArgs &a, const char *what, hipStream_t s) {
  int cus = 0;
  DevInfo di;
  if (device_info(&di) == 0) cus = di.cus;
  hipError_t e = lbk::launch_gemv(fmt, a, cus, s);
  if (e != hipSuccess) return fail_hip(e, what);
  return ok(LB_ISA_GFX950);
}

}  // namespace

extern "C" {

int lbd_gemv_w4a16_fused(const float *x, int M, int Kp, const uint8_t *qw, const float *scales,
                         const uint8_t *zeros, int N, float *y, const lbd_fusion *f, void *stream) {
  int rc = check_shape(M, Kp, N, LB_GROUP);
  if (rc < 0) return rc;
  if ((!x && !(f && f->attn_part)) || !qw || !scales || !y) return fail(LB_ERR_ARG, "null pointer");
  if ((x && !aligned16(x)) || !aligned16(qw)) return fail(LB_ERR_ARG, "x and qw must be 16-byte aligned");
  lbk::GemmArgs a;
  a.x = x; a.qw = qw; a.scales = scales; a.zeros = zeros; a.y = y;
  a.M = M; a.Kp = Kp; a.N = N;
  if ((rc = fused_args(lbk::F_W4A16, f, a)) < 0) return rc;
  return run_fused(lbk::F_W4A16, a, "fused W4A16 GEMV launch", static_cast<hipStream_t>(stream));
}

int lbd_gemv_mxfp4_fused(const float *x, int M, int Kp, const uint8_t *qw, const uint8_t *e8m0,
                         int N, float *y, const lbd_fusion *f, void *stream) {
  int rc = check_shape(M, Kp, N, LB_MXBLOCK);
  if (rc < 0) return rc;
  if ((!x && !(f && f->attn_part)) || !qw || !e8m0 || !y) return fail(LB_ERR_ARG, "null pointer");
  if ((x && !aligned16(x)) || !aligned16(qw)) return fail(LB_ERR_ARG, "x and qw must be 16-byte aligned");
  lbk::GemmArgs a;
  a.x = x; a.qw = qw; a.e8m0 = e8m0; a.y = y;
  a.M = M; a.Kp = Kp; a.N = N;
  if ((rc = fused_args(lbk::F_MXFP4, f, a)) < 0) return rc;
  return run_fused(lbk::F_MXFP4, a, "fused MXFP4 GEMV launch", static_cast<hipStream_t>(stream));
}

int lbd_gemv_w4a8_fused(const float *x, int M, int Kp, const uint8_t *qw, const float *scales,
                        const uint8_t *zeros, int N, float *y, const lbd_fusion *f, void *stream) {
  int rc = check_shape(M, Kp, N, LB_GROUP);
  if (rc < 0) return rc;
  if ((!x && !(f && f->attn_part)) || !qw || !scales || !y) return fail(LB_ERR_ARG, "null pointer");
  if ((x && !aligned16(x)) || !aligned16(qw)) return fail(LB_ERR_ARG, "x and qw must be 16-byte aligned");
  lbk::GemmArgs a;
  a.x = x; a.qw = qw; a.scales = scales; a.zeros = zeros; a.y = y;
  a.M = M; a.Kp = Kp; a.N = N;
  if ((rc = fused_args(lbk::F_W4A8, f, a)) < 0) return rc;
  return run_fused(lbk::F_W4A8, a, "fused W4A8 GEMV launch", static_cast<hipStream_t>(stream));
}

}  // extern "C"

namespace {

// Group-32 int4 GEMMs: the small-M kernels over slices of at most four activation
// rows (every slice reads the weights again; there is no matrix-core path for
// groups of 32).
int run_g32(int fmt, const lbk::GemmArgs &a0, hipStream_t s) {
  int mb = 0;
  const int nit = ((a0.Kp >> 5) + 63) / 64;
  for (int m = 4; m >= 1 && !mb; m--) {
    const bool fp32_rows = fmt == lbk::F_W4A16G32 && m >= 2 && nit > 4;  // no such instantiation
    if (!fp32_rows && lbk::gemv_eligible(fmt, m, a0.Kp)) mb = m;
  }
  if (!mb) return fail(LB_ERR_SHAPE, "group-32 GEMMs take Kp up to 14336 (W4A16) / 16384 (W4A8)");
  int cus = 0;
  DevInfo di;
  if (device_info(&di) == 0) cus = di.cus;
  for (int m0 = 0; m0 < a0.M; m0 += mb) {
    lbk::GemmArgs a = a0;
    a.x = a0.x + (size_t)m0 * a0.Kp;
    a.y = a0.y + (size_t)m0 * a0.N;
    a.M = std::min(mb, a0.M - m0);
    hipError_t e = lbk::launch_gemv(fmt, a, cus, s);
    if (e != hipSuccess) return fail_hip(e, "group-32 GEMV launch");
  }
  return ok(LB_ISA_GFX950);
}

int g32_args(const float *x, int M, int Kp, const uint8_t *qw, const float *scales, const uint8_t *zeros, int N,
             float *y, lbk::GemmArgs &a) {
  int rc = check_shape(M, Kp, N, LB_G32);
  if (rc < 0) return rc;
  if (!x || !qw || !scales || !y) return fail(LB_ERR_ARG, "null pointer");
  if (!aligned16(x) || !aligned16(qw)) return fail(LB_ERR_ARG, "x and qw must be 16-byte aligned");
  a.x = x; a.qw = qw; a.scales = scales; a.zeros = zeros; a.y = y;
  a.M = M; a.Kp = Kp; a.N = N;
  return 0;
}

}  // namespace

extern "C" {

int lbd_gemm_w4a16_g32(const float *x, int M, int Kp, const uint8_t *qw, const float *scales, const uint8_t *zeros,
                       int N, float *y, void *stream) {
  lbk::GemmArgs a;
  const int rc = g32_args(x, M, Kp, qw, scales, zeros, N, y, a);
  return rc < 0 ? rc : run_g32(lbk::F_W4A16G32, a, static_cast<hipStream_t>(stream));
}

int lbd_gemm_w4a8_g32(const float *x, int M, int Kp, const uint8_t *qw, const float *scales, const uint8_t *zeros,
                      int N, float *y, void *stream) {
  lbk::GemmArgs a;
  const int rc = g32_args(x, M, Kp, qw, scales, zeros, N, y, a);
  return rc < 0 ? rc : run_g32(lbk::F_W4A8G32, a, static_cast<hipStream_t>(stream));
}

int lbd_argmax_finalize(unsigned long long *key, int32_t *tok, int32_t *pos, int inc, int32_t *hist, int hist_len,
                        void *stream) {
  if (!key || !tok) return fail(LB_ERR_ARG, "null pointer");
  LB_LAUNCH(lbk::launch_argmax_finalize(key, tok, pos, inc, hist, hist_len, static_cast<hipStream_t>(stream)),
            "argmax finalize launch");
}

static int attention_decode(const float *qkv, int H, int KV, int D, const float *cos_table, const float *sin_table,
                     const int32_t *pos, int max_pos, float *k_cache, float *v_cache, int cap, float *out, void *work,
                     size_t work_bytes, void *stream) {
  if (H <= 0 || KV <= 0 || H % KV || H / KV > lbk::kAttnMaxGroup || (D != 32 && D != 64 && D != 128) ||
      max_pos <= 0 || cap <= 0 || cap > 16000)
    return fail(LB_ERR_SHAPE, "bad shape");
  if (!qkv || !cos_table || !sin_table || !pos || !k_cache || !v_cache || !out)
    return fail(LB_ERR_ARG, "null pointer");
  if (!aligned16(qkv) || !aligned16(cos_table) || !aligned16(sin_table) || !aligned16(k_cache) ||
      !aligned16(v_cache))
    return fail(LB_ERR_ARG, "qkv, the tables and the caches must be 16-byte aligned");
  if (work && (!aligned16(work) || !aligned16(out)))
    return fail(LB_ERR_ARG, "work and out must be 16-byte aligned");
  if (work && work_bytes < lbk::attn_work_bytes(H, D, cap))
    return fail(LB_ERR_ARG, "work smaller than lbd_attention_decode_work_bytes");
  LB_LAUNCH(lbk::launch_attention_decode(qkv, H, KV, D, cos_table, sin_table, pos, max_pos, k_cache, v_cache, cap,
                                         out, static_cast<float *>(work), static_cast<hipStream_t>(stream)),
            "attention decode launch");
}

int lbd_attention_decode(const float *qkv, int H, int KV, int D, const float *cos_table, const float *sin_table,
                         const int32_t *pos, int max_pos, float *k_cache, float *v_cache, int cap, float *out,
                         void *stream) {
  return attention_decode(qkv, H, KV, D, cos_table, sin_table, pos, max_pos, k_cache, v_cache, cap, out, nullptr, 0,
                          stream);
}

size_t lbd_attention_decode_work_bytes(int H, int D, int cap) {
  if (H <= 0 || (D != 32 && D != 64 && D != 128) || cap <= 0) return 0;
  return lbk::attn_work_bytes(H, D, cap);
}

int lbd_attention_slices(const float *qkv, int H, int KV, int D, const float *cos_table, const float *sin_table,
                         const int32_t *pos, int max_pos, float *k_cache, float *v_cache, int cap, float *part,
                         size_t part_bytes, void *stream) {
  if (H <= 0 || KV <= 0 || H % KV || H / KV > lbk::kAttnMaxGroup || (D != 32 && D != 64 && D != 128) ||
      max_pos <= 0 || cap <= 0 || cap > 16000)
    return fail(LB_ERR_SHAPE, "bad shape");
  if (!qkv || !cos_table || !sin_table || !pos || !k_cache || !v_cache || !part)
    return fail(LB_ERR_ARG, "null pointer");
  if (!aligned16(qkv) || !aligned16(cos_table) || !aligned16(sin_table) || !aligned16(k_cache) ||
      !aligned16(v_cache) || !aligned16(part))
    return fail(LB_ERR_ARG, "qkv, the tables, the caches and part must be 16-byte aligned");
  if (part_bytes < lbk::attn_work_bytes(H, D, cap))
    return fail(LB_ERR_ARG, "part smaller than lbd_attention_decode_work_bytes");
  LB_LAUNCH(lbk::launch_attention_slices(qkv, H, KV, D, cos_table, sin_table, pos, max_pos, k_cache, v_cache, cap,
                                         part, static_cast<hipStream_t>(stream)),
            "attention slices launch");
}

int lbd_attention_merge(const float *part, size_t part_bytes, int H, int D, const int32_t *pos, int cap, float *out,
                        void *stream) {
  if (H <= 0 || (D != 32 && D != 64 && D != 128) || cap <= 0 || cap > 16000) return fail(LB_ERR_SHAPE, "bad shape");
  if (!part || !pos || !out) return fail(LB_ERR_ARG, "null pointer");
  if (!aligned16(part) || !aligned16(out)) return fail(LB_ERR_ARG, "part and out must be 16-byte aligned");
  if (part_bytes < lbk::attn_work_bytes(H, D, cap))
    return fail(LB_ERR_ARG, "part smaller than lbd_attention_decode_work_bytes");
  LB_LAUNCH(lbk::launch_attention_merge(part, H, D, pos, cap, out, static_cast<hipStream_t>(stream)),
            "attention merge launch");
}

int lbd_attention_decode_ws(const float *qkv, int H, int KV, int D, const float *cos_table, const float *sin_table,
                            const int32_t *pos, int max_pos, float *k_cache, float *v_cache, int cap, float *out,
                            void *work, size_t work_bytes, void *stream) {
  return attention_decode(qkv, H, KV, D, cos_table, sin_table, pos, max_pos, k_cache, v_cache, cap, out, work,
                          work_bytes, stream);
}

// ---------------------------------------------------------------- host-pointer GEMMs

int lb_gemm_w4a16(const float *x, int M, int Kp, const uint8_t *qw, const float *scales,
                  const uint8_t *zeros, int N, float *y, const lb_params *p) {
  int rc = check_shape(M, Kp, N, LB_GROUP);
  if (rc < 0) return rc;
  if ((rc = check_params(p, M)) < 0) return rc;
  if (!x || !qw || !scales || !y) return fail(LB_ERR_ARG, "null pointer");
  Ctx *c = nullptr;
  if ((rc = get_ctx(&c)) < 0) return rc;
  const int G = Kp / LB_GROUP;
  const size_t bx = (size_t)M * Kp * 4, bq = (size_t)N * Kp / 2, bs = (size_t)N * G * 4,
               bz = zeros ? (size_t)N * G : 0, by = (size_t)M * N * 4;
  // the matrix-core regime runs the bf16x3 GEMM on a t16 copy repacked on the device
  // in the call (as a resident handle's first matrix-core GEMM does), with room for
  // the K split; shapes past the t16 limits keep the fp32 MFMA kernel
  const bool t16 = choose_path(lbk::F_W4A16, M, Kp, p) == LB_ISA_GFX950_MFMA && host_t16_fits(M, Kp, N);
  const size_t bqt = t16 ? lbk::t16_qw_bytes(N, Kp) : 0, bst = t16 ? lbk::t16_group_entries(N, Kp) * 4 : 0,
               bzt = t16 && zeros ? lbk::t16_group_entries(N, Kp) : 0,
               bw = t16 ? lbd_bf16x3_workspace_bytes_split(0, M, N, Kp) : 0;
  Arena ar;
  const size_t ox = ar.take(bx), oq = ar.take(bq), os = ar.take(bs), oz = ar.take(bz), oy = ar.take(by);
  const size_t oqt = ar.take(bqt), ost = ar.take(bst), ozt = ar.take(bzt), ow = ar.take(bw);
  if ((rc = grow(&c->buf, &c->cap, ar.off, c->stream)) < 0) return rc;
  char *b = c->buf;
  hipStream_t s = c->stream;
  LB_HIP(hipMemcpyAsync(b + ox, x, bx, hipMemcpyHostToDevice, s), "copy x");
  LB_HIP(hipMemcpyAsync(b + oq, qw, bq, hipMemcpyHostToDevice, s), "copy qw");
  LB_HIP(hipMemcpyAsync(b + os, scales, bs, hipMemcpyHostToDevice, s), "copy scales");
  if (zeros) LB_HIP(hipMemcpyAsync(b + oz, zeros, bz, hipMemcpyHostToDevice, s), "copy zeros");
  const auto *dq = reinterpret_cast<uint8_t *>(b + oq);
  const auto *ds = reinterpret_cast<float *>(b + os);
  const auto *dz = zeros ? reinterpret_cast<uint8_t *>(b + oz) : nullptr;
  if (t16) {
    auto *qt = reinterpret_cast<uint8_t *>(b + oqt), *zt = zeros ? reinterpret_cast<uint8_t *>(b + ozt) : nullptr;
    auto *st = reinterpret_cast<float *>(b + ost);
    if ((rc = lbd_repack_int4_t16(dq, ds, dz, N, Kp, qt, st, zt, s)) < 0) return rc;
    rc = lbd_gemm_w4a16_t16(reinterpret_cast<float *>(b + ox), M, Kp, qt, st, zt, N,
                            reinterpret_cast<float *>(b + oy), p, b + ow, bw, s);
  } else {
    rc = lbd_gemm_w4a16(reinterpret_cast<float *>(b + ox), M, Kp, dq, ds, dz, N, reinterpret_cast<float *>(b + oy),
                        p, s);
  }
  if (rc < 0) return rc;
  LB_HIP(hipMemcpyAsync(y, b + oy, by, hipMemcpyDeviceToHost, s), "copy y");
  LB_HIP(hipStreamSynchronize(s), "synchronize");
  return ok(rc);
}

int lb_gemm_mxfp4(const float *x, int M, int Kp, const uint8_t *qw, const uint8_t *e8m0, int N,
                  float *y, const lb_params *p) {
  int rc = check_shape(M, Kp, N, LB_MXBLOCK);
  if (rc < 0) return rc;
  if ((rc = check_params(p, M)) < 0) return rc;
  if (!x || !qw || !e8m0 || !y) return fail(LB_ERR_ARG, "null pointer");
  Ctx *c = nullptr;
  if ((rc = get_ctx(&c)) < 0) return rc;
  const size_t bx = (size_t)M * Kp * 4, bq = (size_t)N * Kp / 2, be = (size_t)N * (Kp / LB_MXBLOCK),
               by = (size_t)M * N * 4;
  // as lb_gemm_w4a16: the matrix-core regime repacks to t16 and runs bf16x3
  const bool t16 = choose_path(lbk::F_MXFP4, M, Kp, p) == LB_ISA_GFX950_MFMA && host_t16_fits(M, Kp, N);
  const size_t bqt = t16 ? lbk::t16_qw_bytes(N, Kp) : 0, bet = t16 ? lbk::t16_e8m0_bytes(N, Kp) : 0,
               bw = t16 ? lbd_bf16x3_workspace_bytes_split(1, M, N, Kp) : 0;
  Arena ar;
  const size_t ox = ar.take(bx), oq = ar.take(bq), oe = ar.take(be), oy = ar.take(by);
  const size_t oqt = ar.take(bqt), oet = ar.take(bet), ow = ar.take(bw);
  if ((rc = grow(&c->buf, &c->cap, ar.off, c->stream)) < 0) return rc;
  char *b = c->buf;
  hipStream_t s = c->stream;
  LB_HIP(hipMemcpyAsync(b + ox, x, bx, hipMemcpyHostToDevice, s), "copy x");
  LB_HIP(hipMemcpyAsync(b + oq, qw, bq, hipMemcpyHostToDevice, s), "copy qw");
  LB_HIP(hipMemcpyAsync(b + oe, e8m0, be, hipMemcpyHostToDevice, s), "copy e8m0");
  const auto *dq = reinterpret_cast<uint8_t *>(b + oq), *de = reinterpret_cast<uint8_t *>(b + oe);
  if (t16) {
    auto *qt = reinterpret_cast<uint8_t *>(b + oqt), *et = reinterpret_cast<uint8_t *>(b + oet);
    if ((rc = lbd_repack_mxfp4_t16(dq, de, N, Kp, qt, et, s)) < 0) return rc;
    rc = lbd_gemm_mxfp4_t16(reinterpret_cast<float *>(b + ox), M, Kp, qt, et, N, reinterpret_cast<float *>(b + oy),
                            p, b + ow, bw, s);
  } else {
    rc = lbd_gemm_mxfp4(reinterpret_cast<float *>(b + ox), M, Kp, dq, de, N, reinterpret_cast<float *>(b + oy), p, s);
  }
  if (rc < 0) return rc;
  LB_HIP(hipMemcpyAsync(y, b + oy, by, hipMemcpyDeviceToHost, s), "copy y");
  LB_HIP(hipStreamSynchronize(s), "synchronize");
  return ok(rc);
}

int lb_gemm_w4a8(const float *x, int M, int Kp, const uint8_t *qw, const float *scales,
                 const uint8_t *zeros, int N, float *y, const lb_params *p) {
  int rc = check_shape(M, Kp, N, LB_GROUP);
  if (rc < 0) return rc;
  if ((rc = check_params(p, M)) < 0) return rc;
  if (!x || !qw || !scales || !y) return fail(LB_ERR_ARG, "null pointer");
  Ctx *c = nullptr;
  if ((rc = get_ctx(&c)) < 0) return rc;
  const int G = Kp / LB_GROUP;
  const size_t bx = (size_t)M * Kp * 4, bq = (size_t)N * Kp / 2, bs = (size_t)N * G * 4,
               bz = zeros ? (size_t)N * G : 0, by = (size_t)M * N * 4, bw = w4a8_ws_bytes(M, Kp);
  Arena ar;
  const size_t ox = ar.take(bx), oq = ar.take(bq), os = ar.take(bs), oz = ar.take(bz), oy = ar.take(by),
               ow = ar.take(bw);
  if ((rc = grow(&c->buf, &c->cap, ar.off, c->stream)) < 0) return rc;
  char *b = c->buf;
  hipStream_t s = c->stream;
  LB_HIP(hipMemcpyAsync(b + ox, x, bx, hipMemcpyHostToDevice, s), "copy x");
  LB_HIP(hipMemcpyAsync(b + oq, qw, bq, hipMemcpyHostToDevice, s), "copy qw");
  LB_HIP(hipMemcpyAsync(b + os, scales, bs, hipMemcpyHostToDevice, s), "copy scales");
  if (zeros) LB_HIP(hipMemcpyAsync(b + oz, zeros, bz, hipMemcpyHostToDevice, s), "copy zeros");
  rc = lbd_gemm_w4a8(reinterpret_cast<float *>(b + ox), M, Kp, reinterpret_cast<uint8_t *>(b + oq),
                     reinterpret_cast<float *>(b + os), zeros ? reinterpret_cast<uint8_t *>(b + oz) : nullptr, N,
                     reinterpret_cast<float *>(b + oy), p, b + ow, bw, s);
  if (rc < 0) return rc;
  LB_HIP(hipMemcpyAsync(y, b + oy, by, hipMemcpyDeviceToHost, s), "copy y");
  LB_HIP(hipStreamSynchronize(s), "synchronize");
  return ok(rc);
}

int lb_gemm_w4a8_q(const int8_t *xq, const float *xs, const int32_t *asum, int M, int Kp,
                   const uint8_t *qw, const float *scales, const uint8_t *zeros, int N, float *y,
                   const lb_params *p) {
  int rc = check_shape(M, Kp, N, LB_GROUP);
  if (rc < 0) return rc;
  if ((rc = check_params(p, M)) < 0) return rc;
  if (!xq || !xs || !asum || !qw || !scales || !y) return fail(LB_ERR_ARG, "null pointer");
  Ctx *c = nullptr;
  if ((rc = get_ctx(&c)) < 0) return rc;
  const int G = Kp / LB_GROUP;
  const size_t bxq = (size_t)M * Kp, bxs = (size_t)M * 4, ba = (size_t)M * G * 4, bq = (size_t)N * Kp / 2,
               bs = (size_t)N * G * 4, bz = zeros ? (size_t)N * G : 0, by = (size_t)M * N * 4;
  Arena ar;
  const size_t oxq = ar.take(bxq), oxs = ar.take(bxs), oa = ar.take(ba), oq = ar.take(bq), os = ar.take(bs),
               oz = ar.take(bz), oy = ar.take(by);
  if ((rc = grow(&c->buf, &c->cap, ar.off, c->stream)) < 0) return rc;
  char *b = c->buf;
  hipStream_t s = c->stream;
  LB_HIP(hipMemcpyAsync(b + oxq, xq, bxq, hipMemcpyHostToDevice, s), "copy xq");
  LB_HIP(hipMemcpyAsync(b + oxs, xs, bxs, hipMemcpyHostToDevice, s), "copy xs");
  LB_HIP(hipMemcpyAsync(b + oa, asum, ba, hipMemcpyHostToDevice, s), "copy asum");
  LB_HIP(hipMemcpyAsync(b + oq, qw, bq, hipMemcpyHostToDevice, s), "copy qw");
  LB_HIP(hipMemcpyAsync(b + os, scales, bs, hipMemcpyHostToDevice, s), "copy scales");
  if (zeros) LB_HIP(hipMemcpyAsync(b + oz, zeros, bz, hipMemcpyHostToDevice, s), "copy zeros");
  rc = lbd_gemm_w4a8_q(reinterpret_cast<int8_t *>(b + oxq), reinterpret_cast<float *>(b + oxs),
                       reinterpret_cast<int32_t *>(b + oa), M, Kp, reinterpret_cast<uint8_t *>(b + oq),
                       reinterpret_cast<float *>(b + os), zeros ? reinterpret_cast<uint8_t *>(b + oz) : nullptr,
                       N, reinterpret_cast<float *>(b + oy), p, s);
  if (rc < 0) return rc;
  LB_HIP(hipMemcpyAsync(y, b + oy, by, hipMemcpyDeviceToHost, s), "copy y");
  LB_HIP(hipStreamSynchronize(s), "synchronize");
  return ok(rc);
}

void lb_quant_act_int8(const float *x, int M, int Kp, int8_t *xq, float *xs, int32_t *asum) {
  if (M <= 0 || Kp <= 0 || Kp % LB_GROUP) {
    fail(LB_ERR_SHAPE, "bad shape");
    return;
  }
  if (!x || !xq || !xs || !asum) {
    fail(LB_ERR_ARG, "null pointer");
    return;
  }
  Ctx *c = nullptr;
  if (get_ctx(&c) < 0) return;
  const int G = Kp / LB_GROUP;
  const size_t bx = (size_t)M * Kp * 4, bxq = (size_t)M * Kp, bxs = (size_t)M * 4, ba = (size_t)M * G * 4;
  Arena ar;
  const size_t ox = ar.take(bx), oxq = ar.take(bxq), oxs = ar.take(bxs), oa = ar.take(ba);
  if (grow(&c->buf, &c->cap, ar.off, c->stream) < 0) return;
  char *b = c->buf;
  hipStream_t s = c->stream;
  hipError_t e;
  if ((e = hipMemcpyAsync(b + ox, x, bx, hipMemcpyHostToDevice, s)) != hipSuccess) { fail_hip(e, "copy x"); return; }
  if (lbd_quant_act_int8(reinterpret_cast<float *>(b + ox), M, Kp, reinterpret_cast<int8_t *>(b + oxq),
                         reinterpret_cast<float *>(b + oxs), reinterpret_cast<int32_t *>(b + oa), s) < 0)
    return;
  if ((e = hipMemcpyAsync(xq, b + oxq, bxq, hipMemcpyDeviceToHost, s)) != hipSuccess) { fail_hip(e, "copy xq"); return; }
  if ((e = hipMemcpyAsync(xs, b + oxs, bxs, hipMemcpyDeviceToHost, s)) != hipSuccess) { fail_hip(e, "copy xs"); return; }
  if ((e = hipMemcpyAsync(asum, b + oa, ba, hipMemcpyDeviceToHost, s)) != hipSuccess) { fail_hip(e, "copy asum"); return; }
  if ((e = hipStreamSynchronize(s)) != hipSuccess) { fail_hip(e, "synchronize"); return; }
  ok(0);
}

int lb_w4a8_group_acc(const int8_t *xq, const int32_t *asum, int M, int Kp, const uint8_t *qw,
                      const uint8_t *zeros, int N, int32_t *out, int isa) {
  int rc = check_shape(M, Kp, N, LB_GROUP);
  if (rc < 0) return rc;
  if (!xq || !asum || !qw || !out) return fail(LB_ERR_ARG, "null pointer");
  Ctx *c = nullptr;
  if ((rc = get_ctx(&c)) < 0) return rc;
  const int G = Kp / LB_GROUP;
  const size_t bxq = (size_t)M * Kp, ba = (size_t)M * G * 4, bq = (size_t)N * Kp / 2, bz = zeros ? (size_t)N * G : 0,
               bo = (size_t)M * N * G * 4;
  Arena ar;
  const size_t oxq = ar.take(bxq), oa = ar.take(ba), oq = ar.take(bq), oz = ar.take(bz), oo = ar.take(bo);
  if ((rc = grow(&c->buf, &c->cap, ar.off, c->stream)) < 0) return rc;
  char *b = c->buf;
  hipStream_t s = c->stream;
  LB_HIP(hipMemcpyAsync(b + oxq, xq, bxq, hipMemcpyHostToDevice, s), "copy xq");
  LB_HIP(hipMemcpyAsync(b + oa, asum, ba, hipMemcpyHostToDevice, s), "copy asum");
  LB_HIP(hipMemcpyAsync(b + oq, qw, bq, hipMemcpyHostToDevice, s), "copy qw");
  if (zeros) LB_HIP(hipMemcpyAsync(b + oz, zeros, bz, hipMemcpyHostToDevice, s), "copy zeros");
  rc = lbd_w4a8_group_acc(reinterpret_cast<int8_t *>(b + oxq), reinterpret_cast<int32_t *>(b + oa), M, Kp,
                          reinterpret_cast<uint8_t *>(b + oq), zeros ? reinterpret_cast<uint8_t *>(b + oz) : nullptr,
                          N, reinterpret_cast<int32_t *>(b + oo), isa, s);
  if (rc < 0) return rc;
  LB_HIP(hipMemcpyAsync(out, b + oo, bo, hipMemcpyDeviceToHost, s), "copy out");
  LB_HIP(hipStreamSynchronize(s), "synchronize");
  return ok(rc);
}

}  // extern "C"

// ---------------------------------------------------------------- allocation-free W4A8 (t16)
//
// lbd_gemm_w4a8_t16_noalloc keeps the quantized activations in `scratch`, a
// file-scope device array each GPU holds until the process ends, so the call
// allocates nothing. Host code never passes the array's name to a kernel (on the
// host it is a stand-in, not a device address): the first call on each device takes
// that device's address of it with hipGetSymbolAddress and every later call uses
// the address kept for the device.

namespace {

constexpr size_t kNoAllocScratchBytes = size_t(8) << 20;

}  // namespace

static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

namespace {

std::mutex g_scratch_mu;
std::unordered_map<int, char *> g_scratch;  // device -> that device's address of `scratch`

int scratch_address(char **out) {
  int dev = 0;
  int rc = current_device(&dev);
  if (rc < 0) return rc;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  auto it = g_scratch.find(dev);
  if (it == g_scratch.end()) {
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return fail_hip(e, "hipGetSymbolAddress of the scratch array");
    if (!p) return fail(LB_ERR_HIP, "hipGetSymbolAddress gave no address for the scratch array");
    it = g_scratch.emplace(dev, static_cast<char *>(p)).first;
  }
  *out = it->second;
  return 0;
}

}  // namespace

extern "C" {

size_t lbd_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

int lbd_gemm_w4a8_t16_noalloc(const float *x, int M, int Kp, const uint8_t *qwt, const float *st, const uint8_t *zt,
                              int N, float *y, const lb_params *p, void *stream) {
  int rc = check_w4a8_t16(x, M, Kp, qwt, st, zt, N, y, p);
  if (rc < 0) return rc;
  const size_t need = w4a8_ws_bytes(M, Kp);
  if (need > kNoAllocScratchBytes)
    return fail(LB_ERR_SHAPE, "lbd_gemm_w4a8_t16_noalloc: the quantized activations of this M x Kp need more "
                              "than its 8 MiB scratch (lbd_w4a8_workspace_bytes(M, Kp) must be at most "
                              "lbd_noalloc_scratch_bytes())");
  char *ws = nullptr;
  if ((rc = scratch_address(&ws)) < 0) return rc;
  return run_w4a8(w4a8_t16_args(x, M, Kp, qwt, st, zt, N, y), p, ws, static_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------- plumbing

int lb_dev_malloc(void **ptr, size_t bytes) {
  if (!ptr) return fail(LB_ERR_ARG, "null pointer");
  if (hipMalloc(ptr, bytes ? bytes : 1) != hipSuccess) return fail(LB_ERR_ALLOC, "hipMalloc failed");
  return ok(0);
}
int lb_dev_free(void *ptr) {
  LB_HIP(hipFree(ptr), "hipFree");
  return ok(0);
}
int lb_memcpy_h2d(void *dst, const void *src, size_t bytes) {
  LB_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
  return ok(0);
}
int lb_memcpy_d2h(void *dst, const void *src, size_t bytes) {
  LB_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
  return ok(0);
}
int lb_memcpy_h2d_async(void *dst, const void *src, size_t bytes, void *stream) {
  LB_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, static_cast<hipStream_t>(stream)),
         "hipMemcpyAsync H2D");
  return ok(0);
}
int lb_memcpy_d2h_async(void *dst, const void *src, size_t bytes, void *stream) {
  LB_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, static_cast<hipStream_t>(stream)),
         "hipMemcpyAsync D2H");
  return ok(0);
}
int lb_memcpy_d2d(void *dst, const void *src, size_t bytes) {
  LB_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice), "hipMemcpy D2D");
  return ok(0);
}
int lb_memset_d(void *dst, int value, size_t bytes) {
  LB_HIP(hipMemset(dst, value, bytes), "hipMemset");
  return ok(0);
}
int lb_dev_synchronize(void) {
  LB_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
  return ok(0);
}
int lb_stream_create(void **stream) {
  if (!stream) return fail(LB_ERR_ARG, "null pointer");
  hipStream_t s;
  LB_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
  *stream = s;
  return ok(0);
}
int lb_stream_destroy(void *stream) {
  LB_HIP(hipStreamDestroy(static_cast<hipStream_t>(stream)), "hipStreamDestroy");
  return ok(0);
}
int lb_stream_synchronize(void *stream) {
  LB_HIP(hipStreamSynchronize(static_cast<hipStream_t>(stream)), "hipStreamSynchronize");
  return ok(0);
}
int lb_event_create(void **event) {
  if (!event) return fail(LB_ERR_ARG, "null pointer");
  hipEvent_t e;
  LB_HIP(hipEventCreate(&e), "hipEventCreate");
  *event = e;
  return ok(0);
}
int lb_event_destroy(void *event) {
  LB_HIP(hipEventDestroy(static_cast<hipEvent_t>(event)), "hipEventDestroy");
  return ok(0);
}
int lb_event_record(void *event, void *stream) {
  LB_HIP(hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream)), "hipEventRecord");
  return ok(0);
}
int lb_event_synchronize(void *event) {
  LB_HIP(hipEventSynchronize(static_cast<hipEvent_t>(event)), "hipEventSynchronize");
  return ok(0);
}
int lb_event_elapsed_ms(void *start, void *stop, float *ms) {
  if (!ms) return fail(LB_ERR_ARG, "null pointer");
  LB_HIP(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)),
         "hipEventElapsedTime");
  return ok(0);
}
int lb_stream_begin_capture(void *stream) {
  LB_HIP(hipStreamBeginCapture(static_cast<hipStream_t>(stream), hipStreamCaptureModeThreadLocal),
         "hipStreamBeginCapture");
  return ok(0);
}
int lb_stream_end_capture(void *stream, void **graph_exec) {
  if (!graph_exec) return fail(LB_ERR_ARG, "null pointer");
  hipGraph_t g = nullptr;
  LB_HIP(hipStreamEndCapture(static_cast<hipStream_t>(stream), &g), "hipStreamEndCapture");
  hipGraphExec_t ex = nullptr;
  hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) return fail_hip(e, "hipGraphInstantiate");
  *graph_exec = ex;
  return ok(0);
}
int lb_graph_launch(void *graph_exec, void *stream) {
  LB_HIP(hipGraphLaunch(static_cast<hipGraphExec_t>(graph_exec), static_cast<hipStream_t>(stream)),
         "hipGraphLaunch");
  return ok(0);
}
int lb_graph_destroy(void *graph_exec) {
  LB_HIP(hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph_exec)), "hipGraphExecDestroy");
  return ok(0);
}
int lbd_read_kernel(const void *src, size_t bytes, int workgroups, int threads, int loads, uint32_t *sink,
                    void *stream) {
  if (!src || !sink || !aligned16(src)) return fail(LB_ERR_ARG, "read needs a 16-byte aligned source and a sink");
  if (bytes == 0 || bytes % 16 || bytes > 0xFFFFFFF0u || workgroups <= 0 || workgroups > 65536 ||
      (threads != 256 && threads != 512) || (loads != 1 && loads != 2 && loads != 4 && loads != 8))
    return fail(LB_ERR_ARG, "read: bytes a multiple of 16 below 4 GiB, 1..65536 workgroups of 256 or 512 "
                            "threads, 1/2/4/8 loads");
  hipError_t e = lbk::launch_stream_read(src, bytes, workgroups, threads, loads, sink,
                                         static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail_hip(e, "read kernel launch");
  return ok(0);
}
int lbd_probe_valu(int op, int iters, int workgroups, float *out, void *stream) {
  if (!out) return fail(LB_ERR_ARG, "probe needs an output buffer");
  if (op < 0 || op >= lbk::valu_probe_forms() || iters <= 0 || workgroups <= 0 || workgroups > 65536)
    return fail(LB_ERR_ARG, "probe: op 0 .. lbd_probe_forms() - 1, iters > 0, 1..65536 workgroups");
  hipError_t e = lbk::launch_valu_probe(op, iters, workgroups, out, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail_hip(e, "probe launch");
  return ok(0);
}
int lbd_probe_forms(void) { return lbk::valu_probe_forms(); }
int lbd_probe_mfma_valu(int variant, int iters, int workgroups, int threads, float *out, void *stream) {
  if (!out) return fail(LB_ERR_ARG, "probe needs an output buffer");
  if (variant < 0 || variant > 3 || iters <= 0 || workgroups <= 0 || workgroups > 65536 ||
      (threads != 256 && threads != 512))
    return fail(LB_ERR_ARG, "probe: variant 0..3, iters > 0, 1..65536 workgroups of 256 or 512 threads");
  hipError_t e = lbk::launch_mfma_valu_probe(variant, iters, workgroups, threads, out,
                                             static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail_hip(e, "probe launch");
  return ok(0);
}
int lbd_empty_kernel(int workgroups, void *stream) {
  if (workgroups <= 0 || workgroups > 65536) return fail(LB_ERR_ARG, "empty kernel: 1..65536 workgroups");
  hipError_t e = lbk::launch_empty(workgroups, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail_hip(e, "empty kernel launch");
  return ok(0);
}
int lbd_probe_div127(uint32_t *out, void *stream) {
  if (!out || (reinterpret_cast<uintptr_t>(out) & 3)) return fail(LB_ERR_ARG, "div127 probe needs two device dwords");
  hipError_t e = lbk::launch_div127_probe(out, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail_hip(e, "div127 probe launch");
  return ok(0);
}
int lbd_probe_grid_barrier(int workgroups, int rounds, int mode, uint32_t *sync, size_t sync_bytes,
                           uint32_t *status, void *stream) {
  if (!sync || !status) return fail(LB_ERR_ARG, "barrier probe needs a sync buffer and a status word");
  if (workgroups <= 0 || workgroups > lbk::kBarrierMaxWorkgroups || rounds < 0 || rounds > 100000 || mode < 0 ||
      mode > 2)
    return fail(LB_ERR_ARG, "barrier probe: 1..1024 workgroups, 0..100000 rounds, mode 0, 1 or 2");
  if (sync_bytes < (size_t)(64 + workgroups) * 4) return fail(LB_ERR_ARG, "barrier probe: sync buffer too small");
  hipError_t e = lbk::launch_grid_barrier(workgroups, rounds, mode, sync, status, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail_hip(e, "barrier probe launch");
  return ok(0);
}
int lbd_copy_kernel(void *dst, const void *src, size_t bytes, void *stream) {
  if (!dst || !src || bytes % 16 || !aligned16(dst) || !aligned16(src))
    return fail(LB_ERR_ARG, "copy needs 16-byte aligned pointers and a multiple of 16 bytes");
  hipError_t e = lbk::launch_copy(dst, src, bytes, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail_hip(e, "copy kernel launch");
  return ok(0);
}

}  // extern "C"
