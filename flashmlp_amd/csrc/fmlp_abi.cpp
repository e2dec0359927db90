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
int io_of(int dtype) { return dtype & ~(FMLP_OUT_F32 | FMLP_DW_HILO); }

int check_shape(int64_t H, int64_t B, int64_t D, int64_t E, int dtype) {
  if (H < 0 || B < 0 || D < 0 || E < 0)
    return fail(FMLP_ERR_INVALID_ARG, "negative dimension (H=%lld B=%lld D=%lld E=%lld)", (long long)H,
                (long long)B, (long long)D, (long long)E);
  const int io = dtype & ~(FMLP_OUT_F32 | FMLP_DW_HILO);
  if (io != FMLP_DTYPE_F16 && io != FMLP_DTYPE_BF16)
    return fail(FMLP_ERR_UNSUPPORTED,
                "dtype code %d: only fp16 (0) and bf16 (1) are supported, optionally with FMLP_OUT_F32 / FMLP_DW_HILO",
                dtype);
  if (D != 64 && D != 128) return fail(FMLP_ERR_UNSUPPORTED, "hidden dimension D=%lld: supported D are 64 and 128", (long long)D);
  if (E < 8 || E % 8 != 0)
    return fail(FMLP_ERR_UNSUPPORTED, "intermediate dimension E=%lld: must be a positive multiple of 8", (long long)E);
  if (B > (1LL << 30) || E > (1LL << 30) || H > (1LL << 30))
    return fail(FMLP_ERR_INVALID_ARG, "dimension too large (H=%lld B=%lld E=%lld)", (long long)H, (long long)B,
                (long long)E);
  // the kernels address one head's W1 / W2 (D x E values) with 32-bit byte offsets
  if (D * E * 2 > 0x7fffffffLL)
    return fail(FMLP_ERR_UNSUPPORTED, "per-head weight slice D*E=%lld values exceeds 2 GiB", (long long)(D * E));
  // every tile count must fit a 32-bit grid
  if (H * ((B + 127) / 128) + H * ((E + 127) / 128) * 64 > 0x7fffffffLL)
    return fail(FMLP_ERR_INVALID_ARG, "problem too large for one launch");
  return FMLP_OK;
}

int check_act(int act) {
  if (act < FMLP_ACT_NONE || act > FMLP_ACT_SIGMOID) return fail(FMLP_ERR_INVALID_ARG, "activation code %d", act);
  return FMLP_OK;
}

int check_ptr(const void* p, const char* name, bool needed) {
  if (!needed) return FMLP_OK;
  if (p == nullptr) return fail(FMLP_ERR_INVALID_ARG, "%s is NULL", name);
  if (!aligned16(p)) return fail(FMLP_ERR_INVALID_ARG, "%s is not 16-byte aligned", name);
  return FMLP_OK;
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

FMLP_EXPORT int fmlp_fwd(const void* x, const void* w1, const void* w2, void* o, int64_t H, int64_t B, int64_t D,
                         int64_t E, int dtype, int act, void* stream) {
  if (dtype & FMLP_DW_HILO) return fail(FMLP_ERR_INVALID_ARG, "FMLP_DW_HILO applies to the backward only");
  int st = check_shape(H, B, D, E, dtype);
  if (st) return st;
  if ((st = check_act(act))) return st;
  const bool rows = H > 0 && B > 0;
  const bool wts = H > 0;
  if ((st = check_ptr(x, "x", rows)) || (st = check_ptr(w1, "w1", wts)) || (st = check_ptr(w2, "w2", wts)) ||
      (st = check_ptr(o, "o", rows)))
    return st;
  if (!rows) return ok();
  fmlp::FwdArgs a{x, w1, w2, o, H, B, D, E, io_of(dtype) == FMLP_DTYPE_BF16, act, (dtype & FMLP_OUT_F32) != 0};
  hipError_t e = fmlp::launch_fwd(a, (hipStream_t)stream);
  if (e != hipSuccess) return fail(FMLP_ERR_HIP, "forward launch: %s", hipGetErrorString(e));
  return ok();
}

FMLP_EXPORT size_t fmlp_bwd_workspace_bytes(int64_t H, int64_t B, int64_t D, int64_t E, int dtype) {
  if (check_shape(H, B, D, E, dtype) != FMLP_OK) return 0;
  int cus = 0;
  if (num_cus_current(&cus) != FMLP_OK) return 0;
  return fmlp::plan_bwd(H, B, D, E, cus).ws_bytes;
}

namespace {

// Argument checks shared by fmlp_bwd and fmlp_bwd_noalloc; fills the plan when there is
// work (returns FMLP_OK with *work = false for H == 0).
int bwd_prepare(const void* x, const void* w1, const void* w2, const void* dout, void* dx, void* dw1, void* dw2,
                int64_t H, int64_t B, int64_t D, int64_t E, int dtype, int act, fmlp::BwdPlan* plan, bool* work) {
  *work = false;
  int st = check_shape(H, B, D, E, dtype);
  if (st) return st;
  if ((st = check_act(act))) return st;
  const bool rows = H > 0 && B > 0;
  const bool wts = H > 0;
  if ((st = check_ptr(x, "x", rows)) || (st = check_ptr(w1, "w1", wts)) || (st = check_ptr(w2, "w2", wts)) ||
      (st = check_ptr(dout, "dout", rows)) || (st = check_ptr(dx, "dx", rows)) || (st = check_ptr(dw1, "dw1", wts)) ||
      (st = check_ptr(dw2, "dw2", wts)))
    return st;
  if (H == 0) return FMLP_OK;
  int cus = 0;
  if ((st = num_cus_current(&cus))) return st;
  *plan = fmlp::plan_bwd(H, B, D, E, cus);
  *work = true;
  return FMLP_OK;
}

}  // namespace

FMLP_EXPORT int fmlp_bwd(const void* x, const void* w1, const void* w2, const void* dout, void* dx, void* dw1,
                         void* dw2, int64_t H, int64_t B, int64_t D, int64_t E, int dtype, int act, void* workspace,
                         size_t workspace_bytes, void* stream) {
  fmlp::BwdPlan plan{};
  bool work = false;
  int st = bwd_prepare(x, w1, w2, dout, dx, dw1, dw2, H, B, D, E, dtype, act, &plan, &work);
  if (st) return st;
  if (!work) return ok();
  if (plan.ws_bytes > 0) {
    if (workspace == nullptr || workspace_bytes < plan.ws_bytes)
      return fail(FMLP_ERR_WORKSPACE, "workspace of %zu bytes given, %zu needed", workspace_bytes, plan.ws_bytes);
    if (!aligned16(workspace)) return fail(FMLP_ERR_INVALID_ARG, "workspace is not 16-byte aligned");
  }
  fmlp::BwdArgs a{x, w1, w2, dout, dx, dw1, dw2, H, B, D, E, io_of(dtype) == FMLP_DTYPE_BF16, act, workspace,
                  (dtype & FMLP_OUT_F32) != 0, (dtype & FMLP_DW_HILO) != 0};
  hipError_t e = fmlp::launch_bwd(a, plan, (hipStream_t)stream);
  if (e != hipSuccess) return fail(FMLP_ERR_HIP, "backward launch: %s", hipGetErrorString(e));
  return ok();
}

FMLP_EXPORT int fmlp_bwd_noalloc(const void* x, const void* w1, const void* w2, const void* dout, void* dx, void* dw1,
                                 void* dw2, int64_t H, int64_t B, int64_t D, int64_t E, int dtype, int act,
                                 void* stream) {
  fmlp::BwdPlan plan{};
  bool work = false;
  int st = bwd_prepare(x, w1, w2, dout, dx, dw1, dw2, H, B, D, E, dtype, act, &plan, &work);
  if (st) return st;
  if (!work) return ok();
  void* scratch = nullptr;
  if (plan.ws_bytes > 0) {
    if (plan.ws_bytes > fmlp::kScratchBytes)
      return fail(FMLP_ERR_WORKSPACE,
                  "fmlp_bwd_noalloc: these shapes need %zu bytes of scratch, the static scratch holds %zu "
                  "(FMLP_SCRATCH_MAX_BYTES); call fmlp_bwd with a workspace instead",
                  plan.ws_bytes, fmlp::kScratchBytes);
    hipError_t e = fmlp::scratch_current_device(&scratch);
    if (e != hipSuccess) return fail(FMLP_ERR_HIP, "scratch lookup: %s", hipGetErrorString(e));
  }
  fmlp::BwdArgs a{x, w1, w2, dout, dx, dw1, dw2, H, B, D, E, io_of(dtype) == FMLP_DTYPE_BF16, act, scratch,
                  (dtype & FMLP_OUT_F32) != 0, (dtype & FMLP_DW_HILO) != 0};
  hipError_t e = fmlp::launch_bwd(a, plan, (hipStream_t)stream);
  if (e != hipSuccess) return fail(FMLP_ERR_HIP, "backward launch: %s", hipGetErrorString(e));
  return ok();
}
