// C ABI of libflashmlp.so (declared in include/flashmlp.h): argument validation,
// status reporting and dispatch to the gfx950 kernels. No allocation, no synchronisation.
#include "../../include/flashmlp.h"
#include "fmlp_launch.h"

#include <hip/hip_runtime.h>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

#define FMLP_EXPORT extern "C" __attribute__((visibility("default")))

static_assert(fmlp::kScratchBytes == FMLP_SCRATCH_MAX_BYTES, "scratch size in the header and the library");

int fmlp::env_int(const char* name, int dflt) {
  const char* v = std::getenv(name);
  if (v == nullptr || *v == 0) return dflt;
  return std::atoi(v);
}

hipError_t fmlp::set_lds_once(const void* kernel, int bytes, std::atomic<unsigned long long>& done) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= 64) return hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  const unsigned long long bit = 1ull << dev;
  if (done.load(std::memory_order_acquire) & bit) return hipSuccess;
  e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess) done.fetch_or(bit, std::memory_order_release);
  return e;
}

namespace {

thread_local std::string g_last_error;

int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int status, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return status;
}

int ok() {
  g_last_error.clear();
  return FMLP_OK;
}

// Compute-unit count per device, read once (device properties do not change).
constexpr int kMaxDevices = 64;
std::atomic<int> g_cus[kMaxDevices];

int num_cus_current(int* out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(FMLP_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(FMLP_ERR_UNSUPPORTED, "device ordinal %d out of range", dev);
  int n = g_cus[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return fail(FMLP_ERR_HIP, "hipDeviceGetAttribute: %s", hipGetErrorString(e));
    if (n <= 0) n = 256;
    g_cus[dev].store(n, std::memory_order_relaxed);
  }
  *out = n;
  return FMLP_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// io dtype of a dtype argument (its flag bits removed)
int io_of(int dtype) {
  return dtype & ~(FMLP_OUT_F32 | FMLP_DW_HILO | FMLP_BWD_RECOMPUTE | FMLP_BWD_STORE_DZ | FMLP_BWD_NO_DX | FMLP_BWD_NO_DW);
}

// backward form selection from the dtype flags (plan_bwd's dz_mode). A backward without dW
// (FMLP_BWD_NO_DW) runs the recompute form's dX programs. One without dX (FMLP_BWD_NO_DX) plans
// as the same call with dX would, and runs that plan's dW programs (E-tile width, B split) alone
// without storing dZ, so its dw1, dw2 are the full call's bit for bit.
int dz_mode_of(int dtype) {
  if (dtype & (FMLP_BWD_RECOMPUTE | FMLP_BWD_NO_DW)) return fmlp::DZ_NEVER;
  return (dtype & FMLP_BWD_STORE_DZ) ? fmlp::DZ_FORCE : fmlp::DZ_AUTO;
}

// workspace bytes a tuned backward with these flags needs under plan p: with FMLP_BWD_NO_DX the
// dW programs' fp32 partials alone (no dZ, no split dX tiles), with FMLP_BWD_NO_DW the split
// ragged dX tiles' partials alone (none when the plan does not split them)
size_t plan_ws_bytes(const fmlp::BwdPlan& p, int dtype) {
  if ((dtype & FMLP_BWD_NO_DX) && (dtype & FMLP_BWD_NO_DW)) return 0;  // nothing to compute
  if (dtype & FMLP_BWD_NO_DW) return p.n_dxs > 0 ? p.ws_bytes - p.dxs_off : 0;
  return (dtype & FMLP_BWD_NO_DX) ? p.dw_ws_bytes : p.ws_bytes;
}
size_t elem_bytes(int io) { return io == FMLP_DTYPE_F32 ? 4 : 2; }

// The tuned kernels (fmlp_fwd.hip, fmlp_bwd.hip) take 16-bit io, D in {64, 128} and
// E % 8 == 0 on dense, 16-byte aligned tensors; everything else within check_shape runs on the
// generic kernels (fmlp_gen.hip).
bool tuned_shape(int64_t D, int64_t E, int io) {
  return (io == FMLP_DTYPE_F16 || io == FMLP_DTYPE_BF16) && (D == 64 || D == 128) && E % 8 == 0;
}
// the tuned forward also takes D = 256 (one wave per SIMD), and so do the backward's D = 256 dX
// and dW programs (launch_dx256, launch_dw256), with the generic kernels' workspace rule
bool fwd_tuned_shape(int64_t D, int64_t E, int io) {
  return tuned_shape(D, E, io) || ((io == FMLP_DTYPE_F16 || io == FMLP_DTYPE_BF16) && D == 256 && E % 8 == 0);
}

int check_shape(int64_t H, int64_t B, int64_t D, int64_t E, int dtype) {
  if (H < 0 || B < 0 || D < 0 || E < 0)
    return fail(FMLP_ERR_INVALID_ARG, "negative dimension (H=%lld B=%lld D=%lld E=%lld)", (long long)H,
                (long long)B, (long long)D, (long long)E);
  const int io = io_of(dtype);
  if (io != FMLP_DTYPE_F16 && io != FMLP_DTYPE_BF16 && io != FMLP_DTYPE_F32)
    return fail(FMLP_ERR_UNSUPPORTED,
                "dtype code %d: fp16 (0), bf16 (1) or fp32 (2), optionally with FMLP_OUT_F32 / FMLP_DW_HILO / "
                "FMLP_BWD_RECOMPUTE or FMLP_BWD_STORE_DZ", dtype);
  if ((dtype & FMLP_BWD_RECOMPUTE) && (dtype & FMLP_BWD_STORE_DZ))
    return fail(FMLP_ERR_INVALID_ARG, "FMLP_BWD_RECOMPUTE and FMLP_BWD_STORE_DZ exclude each other");
  if (!fmlp::gen_supports_d(D))
    return fail(FMLP_ERR_UNSUPPORTED, "hidden dimension D=%lld: supported D are 16, 32, 64, 128 and 256", (long long)D);
  if (E < 1) return fail(FMLP_ERR_UNSUPPORTED, "intermediate dimension E=%lld: must be positive", (long long)E);
  if (B > (1LL << 30) || E > (1LL << 30) || H > (1LL << 30))
    return fail(FMLP_ERR_INVALID_ARG, "dimension too large (H=%lld B=%lld E=%lld)", (long long)H, (long long)B,
                (long long)E);
  // the tuned kernels address one head's W1 / W2 (D x E values) with 32-bit byte offsets
  if (D * E * 4 > 0x7fffffffLL)
    return fail(FMLP_ERR_UNSUPPORTED, "per-head weight slice D*E=%lld values exceeds 512 Mi", (long long)(D * E));
  // every tile count must fit a 32-bit grid
  if (H * ((B + 127) / 128) + H * ((E + 31) / 32) * 64 > 0x7fffffffLL)
    return fail(FMLP_ERR_INVALID_ARG, "problem too large for one launch");
  return FMLP_OK;
}

int check_act(int act) {
  if (act < FMLP_ACT_NONE || act > FMLP_ACT_SIGMOID) return fail(FMLP_ERR_INVALID_ARG, "activation code %d", act);
  return FMLP_OK;
}

// non-NULL and aligned to `align` bytes (16 for the tuned kernels' vector accesses, the
// element size for the generic kernels)
int check_ptr(const void* p, const char* name, bool needed, size_t align = 16) {
  if (!needed) return FMLP_OK;
  if (p == nullptr) return fail(FMLP_ERR_INVALID_ARG, "%s is NULL", name);
  if ((reinterpret_cast<uintptr_t>(p) % align) != 0)
    return fail(FMLP_ERR_INVALID_ARG, "%s is not %zu-byte aligned", name, align);
  return FMLP_OK;
}

// Dense element strides of (n0, n1, n2) row-major.
void dense3(int64_t n1, int64_t n2, long long* s) {
  s[0] = (long long)(n1 * n2);
  s[1] = (long long)n2;
  s[2] = 1;
}
bool is_dense3(const int64_t* s, int64_t n1, int64_t n2) {
  return s[0] == n1 * n2 && s[1] == n2 && s[2] == 1;
}
int check_strides(const int64_t* s, const char* name) {
  if (s == nullptr) return fail(FMLP_ERR_INVALID_ARG, "%s strides are NULL", name);
  for (int i = 0; i < 3; ++i)
    if (s[i] < 0) return fail(FMLP_ERR_INVALID_ARG, "%s stride %d is negative (%lld)", name, i, (long long)s[i]);
  return FMLP_OK;
}

fmlp::GenArgs gen_args(const void* x, const void* w1, const void* w2, const void* dout, void* o, void* dx, void* dw1,
                       void* dw2, int64_t H, int64_t B, int64_t D, int64_t E, int dtype, int act) {
  fmlp::GenArgs g{};
  g.x = x;
  g.w1 = w1;
  g.w2 = w2;
  g.dout = dout;
  g.o = o;
  g.dx = dx;
  g.dw1 = dw1;
  g.dw2 = dw2;
  g.H = H;
  g.B = B;
  g.D = D;
  g.E = E;
  dense3(B, D, g.sx);
  dense3(D, E, g.sw1);
  dense3(E, D, g.sw2);
  dense3(B, D, g.sdo);
  g.io = io_of(dtype) == FMLP_DTYPE_F32 ? fmlp::IO_F32 : io_of(dtype) == FMLP_DTYPE_BF16 ? fmlp::IO_BF16 : fmlp::IO_F16;
  g.act = act;
  g.out_f32 = (dtype & FMLP_OUT_F32) ? 1 : 0;
  g.hilo = (dtype & FMLP_DW_HILO) ? 1 : 0;
  return g;
}

// 16-bit rows whose runs of 8 columns starting at multiples of 8 are aligned 16-byte vectors:
// unit column stride, head and row strides multiples of 8 elements, 16-byte aligned base
int vec_rows(const void* p, const long long* s, int io) {
  if (io == FMLP_DTYPE_F32 || p == nullptr) return 0;
  return (s[2] == 1 && s[1] % 8 == 0 && s[0] % 8 == 0 && aligned16(p)) ? 1 : 0;
}
// the same for runs of 4 columns starting at multiples of 4 (8-byte vectors)
int vec_runs4(const void* p, const long long* s, int io) {
  if (io == FMLP_DTYPE_F32 || p == nullptr) return 0;
  return (s[2] == 1 && s[1] % 4 == 0 && s[0] % 4 == 0 && (reinterpret_cast<uintptr_t>(p) & 7u) == 0) ? 1 : 0;
}

}  // namespace

FMLP_EXPORT int fmlp_abi_version(void) { return FMLP_ABI_VERSION; }

FMLP_EXPORT const char* fmlp_status_string(int status) {
  switch (status) {
    case FMLP_OK: return "ok";
    case FMLP_ERR_INVALID_ARG: return "invalid argument";
    case FMLP_ERR_UNSUPPORTED: return "unsupported configuration";
    case FMLP_ERR_HIP: return "HIP runtime error";
    case FMLP_ERR_WORKSPACE: return "workspace too small";
    default: return "unknown status";
  }
}

FMLP_EXPORT const char* fmlp_last_error(void) { return g_last_error.c_str(); }

FMLP_EXPORT int fmlp_act_from_name(const char* name) {
  if (name == nullptr) return FMLP_ACT_NONE;
  if (std::strcmp(name, "silu") == 0) return FMLP_ACT_SILU;
  if (std::strcmp(name, "leaky_relu") == 0) return FMLP_ACT_LEAKY_RELU;
  if (std::strcmp(name, "sigmoid") == 0) return FMLP_ACT_SIGMOID;
  return FMLP_ACT_NONE;
}

FMLP_EXPORT int fmlp_shape_supported(int64_t H, int64_t B, int64_t D, int64_t E, int dtype) {
  std::string saved = g_last_error;
  const int st = check_shape(H, B, D, E, dtype);
  g_last_error = saved;
  return st == FMLP_OK ? 1 : 0;
}

FMLP_EXPORT int fmlp_shape_tuned(int64_t D, int64_t E, int dtype) { return tuned_shape(D, E, io_of(dtype)) ? 1 : 0; }

namespace {

int fwd_impl(const void* x, const void* w1, const void* w2, void* o, int64_t H, int64_t B, int64_t D, int64_t E,
             const int64_t* sx, const int64_t* sw1, const int64_t* sw2, int dtype, int act, void* ws, size_t ws_bytes,
             void* stream) {
  if (dtype & FMLP_DW_HILO) return fail(FMLP_ERR_INVALID_ARG, "FMLP_DW_HILO applies to the backward only");
  if (dtype & (FMLP_BWD_RECOMPUTE | FMLP_BWD_STORE_DZ | FMLP_BWD_NO_DX | FMLP_BWD_NO_DW))
    return fail(FMLP_ERR_INVALID_ARG,
                "FMLP_BWD_RECOMPUTE / FMLP_BWD_STORE_DZ / FMLP_BWD_NO_DX / FMLP_BWD_NO_DW apply to the backward only");
  int st = check_shape(H, B, D, E, dtype);
  if (st) return st;
  if ((st = check_act(act))) return st;
  if (sx && ((st = check_strides(sx, "x")) || (st = check_strides(sw1, "w1")) || (st = check_strides(sw2, "w2"))))
    return st;
  const bool rows = H > 0 && B > 0;
  const bool wts = H > 0;
  const int io = io_of(dtype);
  const size_t es = elem_bytes(io);
  if ((st = check_ptr(x, "x", rows, es)) || (st = check_ptr(w1, "w1", wts, es)) || (st = check_ptr(w2, "w2", wts, es)) ||
      (st = check_ptr(o, "o", rows, (dtype & FMLP_OUT_F32) ? 4 : es)) || (st = check_ptr(ws, "ws", ws != nullptr)))
    return st;
  if (!rows) return ok();
  const bool dense = sx == nullptr || (is_dense3(sx, B, D) && is_dense3(sw1, D, E) && is_dense3(sw2, E, D));
  hipError_t e;
  if (dense && fwd_tuned_shape(D, E, io) && aligned16(x) && aligned16(w1) && aligned16(w2) && aligned16(o)) {
    int cus = 0;
    if ((st = num_cus_current(&cus))) return st;
    fmlp::FwdArgs a{x, w1, w2, o, H, B, D, E, io == FMLP_DTYPE_BF16, act, (dtype & FMLP_OUT_F32) != 0, cus};
    a.ws = ws;
    a.ws_bytes = ws != nullptr ? ws_bytes : 0;
    e = fmlp::launch_fwd(a, (hipStream_t)stream);
  } else {
    fmlp::GenArgs g = gen_args(x, w1, w2, nullptr, o, nullptr, nullptr, nullptr, H, B, D, E, dtype, act);
    if (sx) {
      for (int i = 0; i < 3; ++i) {
        g.sx[i] = sx[i];
        g.sw1[i] = sw1[i];
        g.sw2[i] = sw2[i];
      }
    }
    g.vec_x = vec_rows(x, g.sx, io);
    if ((st = num_cus_current(&g.num_cus))) return st;
    e = fmlp::launch_gen_fwd(g, (hipStream_t)stream);
  }
  if (e != hipSuccess) return fail(FMLP_ERR_HIP, "forward launch: %s", hipGetErrorString(e));
  return ok();
}

}  // namespace

FMLP_EXPORT int fmlp_fwd(const void* x, const void* w1, const void* w2, void* o, int64_t H, int64_t B, int64_t D,
                         int64_t E, int dtype, int act, void* stream) {
  return fwd_impl(x, w1, w2, o, H, B, D, E, nullptr, nullptr, nullptr, dtype, act, nullptr, 0, stream);
}

FMLP_EXPORT size_t fmlp_fwd_workspace_bytes(int64_t H, int64_t B, int64_t D, int64_t E, int dtype) {
  if (check_shape(H, B, D, E, dtype) != FMLP_OK || !fwd_tuned_shape(D, E, io_of(dtype))) return 0;
  int cus = 0;
  if (num_cus_current(&cus) != FMLP_OK) return 0;
  return fmlp::fwd_plan(H, B, D, E, cus, (size_t)-1).ws_bytes;
}

FMLP_EXPORT int fmlp_fwd_ws(const void* x, const void* w1, const void* w2, void* o, int64_t H, int64_t B, int64_t D,
                            int64_t E, int dtype, int act, void* workspace, size_t workspace_bytes, void* stream) {
  return fwd_impl(x, w1, w2, o, H, B, D, E, nullptr, nullptr, nullptr, dtype, act, workspace, workspace_bytes,
                  stream);
}

FMLP_EXPORT int fmlp_fwd_strided(const void* x, const void* w1, const void* w2, void* o, int64_t H, int64_t B,
                                 int64_t D, int64_t E, const int64_t* x_strides, const int64_t* w1_strides,
                                 const int64_t* w2_strides, int dtype, int act, void* stream) {
  if (x_strides == nullptr || w1_strides == nullptr || w2_strides == nullptr)
    return fail(FMLP_ERR_INVALID_ARG, "stride arrays must not be NULL");
  return fwd_impl(x, w1, w2, o, H, B, D, E, x_strides, w1_strides, w2_strides, dtype, act, nullptr, 0, stream);
}

FMLP_EXPORT size_t fmlp_bwd_workspace_bytes(int64_t H, int64_t B, int64_t D, int64_t E, int dtype) {
  if (check_shape(H, B, D, E, dtype) != FMLP_OK) return 0;
  // the generic and D = 256 dX programs alone use no workspace
  if ((dtype & FMLP_BWD_NO_DW) && !tuned_shape(D, E, io_of(dtype))) return 0;
  int cus = 0;
  if (num_cus_current(&cus) != FMLP_OK) return 0;
  // the generic kernels: the fp32 partials of their dW programs' B split; dense 16-bit D = 256
  // with E % 8 == 0 runs the D = 256 dW programs, whose split may need more
  if (!tuned_shape(D, E, io_of(dtype))) {
    const size_t g = fmlp::gen_plan(H, B, D, E, cus, (size_t)-1).ws_bytes;
    if (!fwd_tuned_shape(D, E, io_of(dtype))) return g;
    const size_t w = fmlp::plan_dw256(H, B, E, (dtype & FMLP_DW_HILO) != 0, cus, (size_t)-1).ws_bytes;
    return w > g ? w : g;
  }
  // the plan depends on the activation, which this query does not take: the largest over them
  size_t n = 0;
  for (int act = 0; act < 4; ++act) {
    const size_t w =
        plan_ws_bytes(fmlp::plan_bwd(H, B, D, E, act, (dtype & FMLP_DW_HILO) != 0, dz_mode_of(dtype), cus), dtype);
    if (w > n) n = w;
  }
  return n;
}

FMLP_EXPORT int fmlp_bwd_plan(int64_t H, int64_t B, int64_t D, int64_t E, int dtype, int act, int64_t* info,
                              int n_info) {
  int st = check_shape(H, B, D, E, dtype);
  if (st) return st;
  if ((st = check_act(act))) return st;
  if (!fwd_tuned_shape(D, E, io_of(dtype))) return fail(FMLP_ERR_UNSUPPORTED, "the generic kernels have no such plan");
  if (n_info > 0 && info == nullptr) return fail(FMLP_ERR_INVALID_ARG, "info is NULL");
  int cus = 0;
  if ((st = num_cus_current(&cus))) return st;
  if (!tuned_shape(D, E, io_of(dtype))) {
    // D = 256: the dX programs (128 rows each) and the dW programs' split with an unlimited
    // workspace (a call splits B only as far as its workspace holds)
    const bool no_dw = (dtype & FMLP_BWD_NO_DW) != 0, no_dx = (dtype & FMLP_BWD_NO_DX) != 0;
    const fmlp::Dw256Plan w = fmlp::plan_dw256(H, B, E, (dtype & FMLP_DW_HILO) != 0, cus, (size_t)-1);
    const int64_t v[11] = {0, no_dw ? 1 : w.nS, 1, 0, 0, no_dw ? 0 : w.n, no_dx ? 0 : H * ((B + 127) / 128), 0,
                           no_dw ? 0 : (int64_t)w.ws_bytes, act, 128};
    for (int i = 0; i < n_info && i < 11; ++i) info[i] = v[i];
    return ok();
  }
  const fmlp::BwdPlan p = fmlp::plan_bwd(H, B, D, E, act, (dtype & FMLP_DW_HILO) != 0, dz_mode_of(dtype), cus);
  // what a call with these flags launches: the dW programs alone (FMLP_BWD_NO_DX, no dZ stored)
  // or the dX programs alone (FMLP_BWD_NO_DW, with the split of the ragged tiles when the plan
  // splits them)
  const bool no_dw = (dtype & FMLP_BWD_NO_DW) != 0, no_dx = (dtype & FMLP_BWD_NO_DX) != 0;
  const bool part = no_dx || no_dw;
  const int64_t v[11] = {p.dz && !part ? 1 : 0, no_dw ? 1 : p.nS, p.dx_es, no_dx ? 0 : p.dxs_xs,
                         p.dx_first ? 1 : 0, no_dw ? 0 : p.n_dw, no_dx ? 0 : p.n_dx, no_dx ? 0 : p.n_dxs,
                         (int64_t)plan_ws_bytes(p, dtype), act, p.et_w};
  for (int i = 0; i < n_info && i < 11; ++i) info[i] = v[i];
  return ok();
}

FMLP_EXPORT int fmlp_bwd_stores_dz(int64_t H, int64_t B, int64_t D, int64_t E, int dtype, int act) {
  if (check_shape(H, B, D, E, dtype) != FMLP_OK || check_act(act) != FMLP_OK) return 0;
  if (!tuned_shape(D, E, io_of(dtype))) return 0;  // the generic kernels recompute
  int cus = 0;
  if (num_cus_current(&cus) != FMLP_OK) return 0;
  if (dtype & (FMLP_BWD_NO_DX | FMLP_BWD_NO_DW)) return 0;  // a partial backward stores no dZ
  return fmlp::plan_bwd(H, B, D, E, act, (dtype & FMLP_DW_HILO) != 0, dz_mode_of(dtype), cus).dz ? 1 : 0;
}

namespace {

// The backward of every entry point: argument checks, then the tuned kernels (dense, aligned,
// tuned shape; fp32 partials in `ws`, or in the static scratch when `noalloc`) or the
// generic kernels.
int bwd_impl(const void* x, const void* w1, const void* w2, const void* dout, void* dx, void* dw1, void* dw2,
             int64_t H, int64_t B, int64_t D, int64_t E, const int64_t* sx, const int64_t* sw1, const int64_t* sw2,
             const int64_t* sdo, int dtype, int act, void* workspace, size_t workspace_bytes, bool noalloc,
             void* stream) {
  int st = check_shape(H, B, D, E, dtype);
  if (st) return st;
  if ((st = check_act(act))) return st;
  if (sx && ((st = check_strides(sx, "x")) || (st = check_strides(sw1, "w1")) || (st = check_strides(sw2, "w2")) ||
             (st = check_strides(sdo, "dout"))))
    return st;
  const bool rows = H > 0 && B > 0;
  const bool wts = H > 0;
  const bool want_dx = (dtype & FMLP_BWD_NO_DX) == 0, want_dw = (dtype & FMLP_BWD_NO_DW) == 0;
  const int io = io_of(dtype);
  const size_t es = elem_bytes(io), os = (dtype & FMLP_OUT_F32) ? 4 : es;
  if ((st = check_ptr(x, "x", rows, es)) || (st = check_ptr(w1, "w1", wts, es)) || (st = check_ptr(w2, "w2", wts, es)) ||
      (st = check_ptr(dout, "dout", rows, es)) || (st = check_ptr(dx, "dx", rows && want_dx, os)) ||
      (st = check_ptr(dw1, "dw1", wts && want_dw, os)) || (st = check_ptr(dw2, "dw2", wts && want_dw, os)))
    return st;
  if (H == 0 || (!want_dx && !want_dw)) return ok();
  const bool dense = sx == nullptr || (is_dense3(sx, B, D) && is_dense3(sw1, D, E) && is_dense3(sw2, E, D) &&
                                       is_dense3(sdo, B, D));
  const bool aligned = aligned16(x) && aligned16(w1) && aligned16(w2) && aligned16(dout) && aligned16(dx) &&
                       aligned16(dw1) && aligned16(dw2);
  hipError_t e = hipSuccess;
  if (dense && aligned && tuned_shape(D, E, io)) {
    int cus = 0;
    if ((st = num_cus_current(&cus))) return st;
    // with a scratch limit the plan only considers B splits (and the stored-dZ form) whose
    // workspace fits it; the unsplit recompute form needs none, so a plan always exists
    fmlp::BwdPlan plan = fmlp::plan_bwd(H, B, D, E, act, (dtype & FMLP_DW_HILO) != 0, dz_mode_of(dtype), cus,
                                        noalloc ? fmlp::kScratchBytes : (size_t)-1);
    // the dW programs alone (FMLP_BWD_NO_DX) need only their fp32 partials, the dX programs
    // alone (FMLP_BWD_NO_DW) only the split ragged tiles' partials, at the workspace's start
    const size_t ws_need = plan_ws_bytes(plan, dtype);
    if (!want_dw) plan.dxs_off = 0;
    void* ws = ws_need > 0 ? workspace : nullptr;
    if (ws_need > 0) {
      if (noalloc) {
        e = fmlp::scratch_current_device(&ws);
        if (e != hipSuccess) return fail(FMLP_ERR_HIP, "scratch lookup: %s", hipGetErrorString(e));
      } else {
        if (workspace == nullptr || workspace_bytes < ws_need)
          return fail(FMLP_ERR_WORKSPACE, "workspace of %zu bytes given, %zu needed", workspace_bytes, ws_need);
        if (!aligned16(workspace)) return fail(FMLP_ERR_INVALID_ARG, "workspace is not 16-byte aligned");
      }
    }
    fmlp::BwdArgs a{x, w1, w2, dout, dx, dw1, dw2, H, B, D, E, io == FMLP_DTYPE_BF16, act, ws,
                    (dtype & FMLP_OUT_F32) != 0, (dtype & FMLP_DW_HILO) != 0, want_dx, want_dw};
    e = fmlp::launch_bwd(a, plan, (hipStream_t)stream);
  } else if (dense && aligned && fwd_tuned_shape(D, E, io)) {
    // dense 16-bit D = 256 with E % 8 == 0: the D = 256 dX and dW programs; as on the generic
    // kernels, the dW programs split B only as far as the given workspace (or the static
    // scratch) holds their partials
    void* ws = nullptr;
    fmlp::Dw256Plan wp{};
    if (want_dw) {
      int cus = 0;
      if ((st = num_cus_current(&cus))) return st;
      const size_t room = noalloc ? fmlp::kScratchBytes
                                  : (workspace != nullptr && aligned16(workspace) ? workspace_bytes : 0);
      wp = fmlp::plan_dw256(H, B, E, (dtype & FMLP_DW_HILO) != 0, cus, room);
      if (wp.ws_bytes > 0) {
        ws = workspace;
        if (noalloc) {
          e = fmlp::scratch_current_device(&ws);
          if (e != hipSuccess) return fail(FMLP_ERR_HIP, "scratch lookup: %s", hipGetErrorString(e));
        }
      }
    }
    fmlp::BwdArgs a{x, w1, w2, dout, dx, dw1, dw2, H, B, D, E, io == FMLP_DTYPE_BF16, act, ws,
                    (dtype & FMLP_OUT_F32) != 0, (dtype & FMLP_DW_HILO) != 0, want_dx, want_dw};
    if (want_dx) e = fmlp::launch_dx256(a, (hipStream_t)stream);
    if (e == hipSuccess && want_dw) e = fmlp::launch_dw256(a, wp, (hipStream_t)stream);
  } else {
    fmlp::GenArgs g = gen_args(x, w1, w2, dout, nullptr, dx, dw1, dw2, H, B, D, E, dtype, act);
    g.want_dx = want_dx ? 1 : 0;
    g.want_dw = want_dw ? 1 : 0;
    if (sx) {
      for (int i = 0; i < 3; ++i) {
        g.sx[i] = sx[i];
        g.sw1[i] = sw1[i];
        g.sw2[i] = sw2[i];
        g.sdo[i] = sdo[i];
      }
    }
    g.vec_x = vec_rows(x, g.sx, io);
    g.vec_do = vec_rows(dout, g.sdo, io);
    g.vec_w2 = vec_rows(w2, g.sw2, io);
    g.vec_w1 = vec_runs4(w1, g.sw1, io);
    if ((st = num_cus_current(&g.num_cus))) return st;
    if (want_dw && B > 0) {
      // B split of the dW programs within the workspace the caller gave (the static scratch for
      // the no-allocation entry point; none: no split). A call that arrives here with the tuned
      // path's workspace (a strided view of a tuned shape) uses what fits of it.
      int cus = 0;
      if ((st = num_cus_current(&cus))) return st;
      const size_t room = noalloc ? fmlp::kScratchBytes
                                  : (workspace != nullptr && aligned16(workspace) ? workspace_bytes : 0);
      const fmlp::GenPlan gp = fmlp::gen_plan(H, B, D, E, cus, room);
      if (gp.nS > 1) {
        void* ws = workspace;
        if (noalloc) {
          e = fmlp::scratch_current_device(&ws);
          if (e != hipSuccess) return fail(FMLP_ERR_HIP, "scratch lookup: %s", hipGetErrorString(e));
        }
        g.nS = gp.nS;
        g.rows_per_split = gp.rows_per_split;
        g.ws = ws;
      }
    }
    e = fmlp::launch_gen_bwd(g, (hipStream_t)stream);
  }
  if (e != hipSuccess) return fail(FMLP_ERR_HIP, "backward launch: %s", hipGetErrorString(e));
  return ok();
}

}  // namespace

FMLP_EXPORT int fmlp_bwd(const void* x, const void* w1, const void* w2, const void* dout, void* dx, void* dw1,
                         void* dw2, int64_t H, int64_t B, int64_t D, int64_t E, int dtype, int act, void* workspace,
                         size_t workspace_bytes, void* stream) {
  return bwd_impl(x, w1, w2, dout, dx, dw1, dw2, H, B, D, E, nullptr, nullptr, nullptr, nullptr, dtype, act, workspace,
                  workspace_bytes, false, stream);
}

FMLP_EXPORT int fmlp_bwd_strided(const void* x, const void* w1, const void* w2, const void* dout, void* dx, void* dw1,
                                 void* dw2, int64_t H, int64_t B, int64_t D, int64_t E, const int64_t* x_strides,
                                 const int64_t* w1_strides, const int64_t* w2_strides, const int64_t* dout_strides,
                                 int dtype, int act, void* workspace, size_t workspace_bytes, void* stream) {
  if (x_strides == nullptr || w1_strides == nullptr || w2_strides == nullptr || dout_strides == nullptr)
    return fail(FMLP_ERR_INVALID_ARG, "stride arrays must not be NULL");
  return bwd_impl(x, w1, w2, dout, dx, dw1, dw2, H, B, D, E, x_strides, w1_strides, w2_strides, dout_strides, dtype,
                  act, workspace, workspace_bytes, false, stream);
}

FMLP_EXPORT int fmlp_bwd_noalloc(const void* x, const void* w1, const void* w2, const void* dout, void* dx, void* dw1,
                                 void* dw2, int64_t H, int64_t B, int64_t D, int64_t E, int dtype, int act,
                                 void* stream) {
  return bwd_impl(x, w1, w2, dout, dx, dw1, dw2, H, B, D, E, nullptr, nullptr, nullptr, nullptr, dtype, act, nullptr, 0,
                  true, stream);
}
