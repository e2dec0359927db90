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
  int num_cus;   // compute units of the current device
  void* ws = nullptr;   // workspace for split tiles' partials (fwd_plan), or none
  size_t ws_bytes = 0;
};

// Forward work split (fwd_plan): es = E parts inside a workgroup (1, or 2 or 4 at D = 64, 4 with
// nwp = 2 waves per part and 64-row tiles); tiles
// 0 .. n_main - 1 run whole, the last n_split tiles each as xs workgroups of nct E-chunks whose
// fp32 partials take ws_bytes of workspace (0 and n_split = 0 when nothing is split). A split
// needing more than max_ws bytes is not taken.
struct FwdPlan {
  int es;
  int nwp = 0;  // waves per E part (32 rows each): 0 = fwd_waves(D); 2 = 64-row tiles (D = 64, es = 4)
  long long n_main;
  int n_split, xs, nct;
  size_t ws_bytes;
};
FwdPlan fwd_plan(int64_t H, int64_t B, int64_t D, int64_t E, int num_cus, size_t max_ws);

// Backward work decomposition (chosen on the host, see plan_bwd):
//   dW programs: H * nE * nS, each owning an E-tile of 128 columns and a B-range of
//                rows_per_split rows (nS > 1 writes fp32 partials to the workspace).
//   dX programs: H * dx_tiles_per_head, each owning 256 rows.
//   Both 8 waves (two per SIMD), in one launch (bwd_kernel), the longer role first.
//   Stored-dZ form (dz): the dW programs also store dZ to the workspace and dX is a GEMM over
//   it (dxg_kernel), two launches instead of recomputing Z and dH in dX programs.
struct BwdPlan {
  int et_w;            // E-columns per dW program: 128, or 64 (D = 64, with dx_es == 2)
  int nE;              // E-tiles of et_w per head
  int nS;              // B splits for the dW programs
  int rows_per_split;  // multiple of 32
  int dx_tiles_per_head;
  int dx_es;           // dX programs: 1 = 256 rows, all E-chunks; 2 = 128 rows, E in two parts (D = 64)
  int dxs_xs, dxs_nct; // ragged last dX tiles (one per head) split over E: parts and chunks per
                       // part (0: not split; single-launch recompute form only)
  long long n_dxs;     // programs of the split tiles (H dxs_xs)
  size_t dxs_off;      // byte offset of their fp32 partials ([H][dxs_xs][rows][D]) in the workspace
  bool dx_first;       // single-launch order: dX programs before the dW programs
  long long n_dw, n_dx;  // dW programs, whole-tile dX programs
  bool dz;             // stored-dZ form
  int Bp;              // B rounded up to 256 (dZ tiles), stored-dZ form
  int n_xg;            // dxg_kernel workgroups (persistent), stored-dZ form
  size_t dz_off;       // byte offset of dZ in the workspace, stored-dZ form
  size_t ws_bytes;     // fp32 partials when nS > 1, then dZ (H nE 128 Bp io elements) when dz
  size_t dw_ws_bytes;  // the fp32 partials alone (at offset 0): what the dW programs need by themselves
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
  bool want_dx = true;  // false: FMLP_BWD_NO_DX (only the dW programs run)
  bool want_dw = true;  // false: FMLP_BWD_NO_DW (only the dX programs run)
};

// io element types of the generic kernels
enum IoType { IO_F16 = 0, IO_BF16 = 1, IO_F32 = 2 };

// Generic kernels (fmlp_gen.hip): D in {16, 32, 64, 128, 256}, fp16 / bf16 / fp32 io, any E,
// inputs with arbitrary element strides (head, row, column), dense row-major outputs.
struct GenArgs {
  const void* x;
  const void* w1;
  const void* w2;
  const void* dout;
  void* o;
  void* dx;
  void* dw1;
  void* dw2;
  long long H, B, D, E;
  long long sx[3], sw1[3], sw2[3], sdo[3];  // element strides of X (H,B,D), W1 (H,D,E), W2 (H,E,D), dO
  int io;       // IoType
  int act;
  int out_f32;  // outputs as fp32 (FMLP_OUT_F32)
  int hilo;     // dW products with hi/lo terms of h and dZ (FMLP_DW_HILO; 16-bit io)
  int want_dx = 1, want_dw = 1;  // FMLP_BWD_NO_DX / FMLP_BWD_NO_DW clear them
  // rows of X / dO whose 8 consecutive 16-bit columns starting at any multiple of 8 are one
  // aligned 16-byte vector (unit column stride, row and head strides multiples of 8 elements,
  // 16-byte aligned base): set by the host, 16-bit io only
  int vec_x = 0, vec_do = 0;
  // the same for the rows of W2 (H, E, D) along d (16 bytes), and W1 (H, D, E) along e in
  // 8-byte runs (unit column stride, strides multiples of 4 elements, 8-byte aligned base)
  int vec_w2 = 0, vec_w1 = 0;
  // backward B split of the dW programs (gen_plan): nS ranges of rows_per_split rows, fp32 partials
  // in ws ([nS][H][E][D] for dW2, then [nS][H][D][E] for dW1) when nS > 1
  int nS = 1, rows_per_split = 0;
  void* ws = nullptr;
  int num_cus = 256;  // compute units of the current device (the forward / dX E split)
};
struct GenPlan {
  int nS;
  int rows_per_split;
  size_t ws_bytes;
};
// B split of the generic dW programs for a device with num_cus CUs, within max_ws bytes of
// workspace (a split that does not fit is not taken: nS = 1 needs none)
GenPlan gen_plan(int64_t H, int64_t B, int64_t D, int64_t E, int num_cus, size_t max_ws);
hipError_t launch_gen_fwd(const GenArgs& a, hipStream_t st);
hipError_t launch_gen_bwd(const GenArgs& a, hipStream_t st);
bool gen_supports_d(int64_t D);

// act: activation code; hilo: FMLP_DW_HILO; dz_mode: whether the stored-dZ form may be chosen
// (DZ_NEVER: FMLP_BWD_RECOMPUTE, DZ_FORCE: FMLP_BWD_STORE_DZ, whenever the workspace allows);
// max_ws: the largest workspace the caller can provide (fmlp_bwd_noalloc: its static scratch)
enum { DZ_NEVER = 0, DZ_AUTO = 1, DZ_FORCE = 2 };
BwdPlan plan_bwd(int64_t H, int64_t B, int64_t D, int64_t E, int act, bool hilo, int dz_mode, int num_cus,
                 size_t max_ws = (size_t)-1);
hipError_t launch_fwd(const FwdArgs& a, hipStream_t st);
// Sum of split tiles' fp32 partials (fmlp_fwd.hip): tiles of BB rows, T per head; split tile s
// (of n_split, the last n_split in row-block-major order) has xs partial [BB][D] blocks at
// ws + (s xs + p) BB D; its rows (< B) of `out` (H, B, D) get their sum in p order, rounded to
// the io dtype (bf16 or fp16) or fp32 when outf32.
hipError_t launch_tile_reduce(const float* ws, void* out, bool bf16, int B, int D, int BB, int H, int T, int xs,
                              int n_split, int outf32, hipStream_t st);
hipError_t launch_bwd(const BwdArgs& a, const BwdPlan& p, hipStream_t st);
// dX alone at D = 256 (dense 16-bit, E % 8 == 0): the tuned dX programs
hipError_t launch_dx256(const BwdArgs& a, hipStream_t st);
// dW alone at D = 256 (dense 16-bit, E % 8 == 0): n = H nE nS programs (nE E-tiles of 128
// columns, nS B ranges of rows_per_split rows), whose fp32 partials take ws_bytes of workspace
// when nS > 1 (a split needing more than max_ws bytes is not taken)
struct Dw256Plan {
  int nE, nS, rows_per_split;
  long long n;
  size_t ws_bytes;
};
Dw256Plan plan_dw256(int64_t H, int64_t B, int64_t E, bool hilo, int num_cus, size_t max_ws);
hipError_t launch_dw256(const BwdArgs& a, const Dw256Plan& p, hipStream_t st);

// The library's static device scratch (fmlp_bwd_noalloc): its device address on the current
// device, looked up once per device, and its size in bytes.
constexpr size_t kScratchBytes = (size_t)64 << 20;
hipError_t scratch_current_device(void** ptr);

}  // namespace fmlp
