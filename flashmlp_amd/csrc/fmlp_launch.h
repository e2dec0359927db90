// Host-side launch descriptors shared by the C-ABI layer and the kernel translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <atomic>

namespace fmlp {

// Integer tuning override from the environment (tile shapes); `dflt` when unset.
int env_int(const char* name, int dflt);

// Raises `kernel`'s dynamic-LDS limit to `bytes` on the current device, once per device:
// `done` is the caller's per-kernel flag word (bit = device ordinal), so later launches
// skip the runtime call.
hipError_t set_lds_once(const void* kernel, int bytes, std::atomic<unsigned long long>& done);

struct FwdArgs {
  const void* x;
  const void* w1;
  const void* w2;
  void* o;
  int64_t H, B, D, E;
  bool bf16;
  int act;
  bool out_f32;  // outputs as fp32 (FMLP_OUT_F32)
};

// Backward work decomposition (chosen on the host, see plan_bwd):
//   dW programs: H * nE * nS, each owning an E-tile of 128 columns and a B-range of
//                rows_per_split rows (nS > 1 writes fp32 partials to the workspace).
//                8 waves (two per SIMD), dw2_kernel.
//   dX programs: H * dx_tiles_per_head, each owning dx_rows rows.
struct BwdPlan {
  int nE;              // E-tiles of 128 per head
  int nS;              // B splits for the dW programs
  int rows_per_split;  // multiple of 32
  int dx_mt;           // 32-row M-tiles per wave in dX programs (rows per program = 128 * dx_mt)
  int dx_kind;         // 0: 4-wave software-pipelined dX programs (128 rows); 1: 8-wave (256 rows)
  int dx_tiles_per_head;
  long long n_dw, n_dx;
  size_t ws_bytes;     // fp32 partials when nS > 1
};

struct BwdArgs {
  const void* x;
  const void* w1;
  const void* w2;
  const void* dout;
  void* dx;
  void* dw1;
  void* dw2;
  int64_t H, B, D, E;
  bool bf16;
  int act;
  void* ws;
  bool out_f32;  // outputs as fp32 (FMLP_OUT_F32)
  bool dw_hilo;  // dW products with hi/lo terms of h and dZ (FMLP_DW_HILO)
};

BwdPlan plan_bwd(int64_t H, int64_t B, int64_t D, int64_t E, int num_cus);
hipError_t launch_fwd(const FwdArgs& a, hipStream_t st);
hipError_t launch_bwd(const BwdArgs& a, const BwdPlan& p, hipStream_t st);

// The library's static device scratch (fmlp_bwd_noalloc): its device address on the current
// device, looked up once per device, and its size in bytes.
constexpr size_t kScratchBytes = (size_t)64 << 20;
hipError_t scratch_current_device(void** ptr);

}  // namespace fmlp
