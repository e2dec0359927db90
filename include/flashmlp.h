/*
 * flashmlp.h — C ABI of the MI355X-native FlashMLP library (libflashmlp.so).
 *
 * The fused multi-head MLP  O = act(X W1) W2  per head, and its gradients, on gfx950
 * (MI355X) with hand-written HIP kernels. This is the boundary under the Python API
 * (flashmlp_fwd / flashmlp_bwd / FlashMLPFunction / FlashMLP); nothing else calls it.
 *
 * Layouts are the reference's (flashmlp.py:1-14, :453-455, :505-508): contiguous row-major
 *   X, O, dO, dX : (H, B, D)      W1, dW1 : (H, D, E)      W2, dW2 : (H, E, D)
 * (the *_strided entry points take X, W1, W2, dO with arbitrary element strides). Element
 * type of every tensor is the io dtype (fp16, bf16 or fp32, as the reference's io dtype is
 * x's, flashmlp.py:87). All pointers are device pointers on the current HIP device, aligned
 * to their element size. Two kernel sets sit behind the entry points: the tuned gfx950
 * kernels for 16-bit io, D in {64, 128}, E % 8 == 0 on dense 16-byte aligned tensors
 * (fmlp_shape_tuned; with D = 256 kernels of their own for the same io, E and layout), and
 * generic kernels for every other supported shape, dtype and layout.
 * The library never allocates: the caller passes every buffer, including the backward
 * workspace.
 *
 * Calls are asynchronous on the given hipStream_t (NULL = default stream) and never
 * synchronise. The library's only global state is caches of values that never change for a
 * device and shape (CU counts, backward plans, each behind its own lock), the thread-local
 * error string, and fmlp_bwd_noalloc's per-device scratch: every entry point but
 * fmlp_bwd_noalloc is reentrant and may run concurrently on any streams and threads;
 * fmlp_bwd_noalloc calls that overlap on one device race (see there). A non-zero return is
 * one of fmlp_status; fmlp_status_string() names it and fmlp_last_error() (thread-local)
 * says which argument was rejected.
 */
#ifndef FLASHMLP_H_
#define FLASHMLP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FMLP_ABI_VERSION 4  /* 2: FMLP_BWD_NO_DX / FMLP_BWD_NO_DW; 3: fmlp_fwd_ws, fmlp_bwd_plan;
                              4: FMLP_BWD_NO_DX runs the full call's dW plan, FMLP_BWD_NO_DW
                              the full recompute launch's dX programs (a workspace where it
                              splits ragged dX tiles) */

typedef enum {
  FMLP_OK = 0,
  FMLP_ERR_INVALID_ARG = 1, /* shape, pointer, alignment or size out of contract */
  FMLP_ERR_UNSUPPORTED = 2, /* valid but not implemented (dtype or flags, D, E < 1, D*E too large) */
  FMLP_ERR_HIP = 3,         /* the HIP runtime reported an error */
  FMLP_ERR_WORKSPACE = 4    /* workspace smaller than fmlp_bwd_workspace_bytes() */
} fmlp_status;

typedef enum { FMLP_DTYPE_F16 = 0, FMLP_DTYPE_BF16 = 1, FMLP_DTYPE_F32 = 2 } fmlp_dtype;

/* OR-ed into the dtype argument of fmlp_fwd / fmlp_bwd: the outputs (o; dx, dw1, dw2) are
 * written as fp32 arrays of the same shapes, holding the fp32-accumulated sums before their
 * final rounding to the io dtype. Inputs stay in the io dtype. A test and diagnostic
 * variant with no counterpart in the reference: it lets callers check the accumulations
 * against an fp32 emulation of the reference's algorithm at 1e-4 relative. */
#define FMLP_OUT_F32 0x100

/* OR-ed into the dtype argument of fmlp_bwd / fmlp_bwd_noalloc (rejected by fmlp_fwd): the
 * dW products take h and dZ as two io-dtype terms, hi = round(v) and lo = round(v - hi),
 * so dw1 and dw2 carry about twice the io dtype's mantissa bits of h and dZ (dx is
 * unchanged). An accuracy mode with no counterpart in the reference, whose kernel rounds h
 * and dZ to the io dtype before the dW products (flashmlp.py:297-320): for callers that
 * need dW elementwise close to an fp32 computation at large B. It doubles the MFMA work of
 * the dW programs (8u -> 12u executed FLOPs, u = H B D E). */
#define FMLP_DW_HILO 0x200

/* OR-ed into the dtype argument of fmlp_bwd / fmlp_bwd_strided / fmlp_bwd_noalloc /
 * fmlp_bwd_workspace_bytes (rejected by fmlp_fwd): keep the reference's recompute-only
 * backward (flashmlp.py:341-421), whose workspace is at most the fp32 dW partials of a B split,
 * instead of the stored-dZ form the library picks for large shapes (see fmlp_bwd). No
 * counterpart in the reference: for callers that need the backward's memory to stay
 * O(weights). Results agree with the stored-dZ form within rounding (the same cast points). */
#define FMLP_BWD_RECOMPUTE 0x400

/* OR-ed into the dtype argument like FMLP_BWD_RECOMPUTE (not together with it): the
 * stored-dZ form whenever the workspace allows it, whatever the estimate says. A test and
 * diagnostic flag with no counterpart in the reference (it lets a caller run both forms on
 * the same shapes). */
#define FMLP_BWD_STORE_DZ 0x800

/* OR-ed into the dtype argument of fmlp_bwd / fmlp_bwd_strided / fmlp_bwd_noalloc: the caller
 * needs no dx (FMLP_BWD_NO_DX: dx may be NULL and is not written; only the dW programs run, in
 * the plan the same call without the flag takes, storing no dZ, with the fp32 partials of their
 * B split as the only workspace; dw1, dw2 are bit-identical to that call's; on the generic
 * kernels, whose B split follows the workspace given, with the same workspace) or no dw1, dw2
 * (FMLP_BWD_NO_DW: both may be NULL and are not written; only the dX programs of the recompute
 * form run, as in its launch, split ragged last tiles and their sum included, whose fp32
 * partials are the only workspace: fmlp_bwd_workspace_bytes is 0, and `workspace` may be NULL,
 * where the plan splits none; dx is bit-identical to the recompute form's, FMLP_BWD_RECOMPUTE,
 * of the same entry point). No
 * counterpart in the reference, whose backward always computes all three: for autograd callers
 * whose input, or whose weights, need no gradient. Both flags together: nothing to compute. */
#define FMLP_BWD_NO_DX 0x1000
#define FMLP_BWD_NO_DW 0x2000

/* Activation codes; names as in the reference ("", "silu", "leaky_relu", "sigmoid"). */
typedef enum { FMLP_ACT_NONE = 0, FMLP_ACT_SILU = 1, FMLP_ACT_LEAKY_RELU = 2, FMLP_ACT_SIGMOID = 3 } fmlp_act;

/* ABI version of the loaded library (FMLP_ABI_VERSION it was built with). */
int fmlp_abi_version(void);

/* Static description of a status code. */
const char* fmlp_status_string(int status);

/* Detail of the last failing call on this thread ("" if none). */
const char* fmlp_last_error(void);

/* Activation code for a reference activation string. Unknown strings map to
 * FMLP_ACT_NONE, like the reference's if/elif chain (flashmlp.py:140-147). */
int fmlp_act_from_name(const char* name);

/* Shapes the library supports: 1 on success. D in {16, 32, 64, 128, 256} (powers of two
 * >= 16, as the reference's tl.arange(0, D) requires, flashmlp.py:66,186); E >= 1; H, B >= 0;
 * dtype fp16, bf16 or fp32 with optional flags. */
int fmlp_shape_supported(int64_t H, int64_t B, int64_t D, int64_t E, int dtype);

/* 1 when the tuned kernels take these shapes (16-bit io, D in {64, 128}, E % 8 == 0) on dense,
 * 16-byte aligned tensors; other supported shapes, dtypes and layouts run on the generic
 * kernels, except that D = 256 (16-bit io, E % 8 == 0, dense, aligned) also has kernels of
 * its own: the tuned forward and the backward's D = 256 dX and dW programs, which keep the
 * generic kernels' workspace rule. No counterpart in the reference (its Triton kernels are
 * autotuned per shape). */
int fmlp_shape_tuned(int64_t D, int64_t E, int dtype);

/*
 * Forward: o = act(x @ w1) @ w2 per head, fp32 accumulation, act(.) rounded to the io
 * dtype before the second product. Replaces flashmlp_fwd's kernel launch
 * (flashmlp.py:428-477, kernel flashmlp.py:63-158). o is fully overwritten.
 */
int fmlp_fwd(const void* x, const void* w1, const void* w2, void* o, int64_t H, int64_t B, int64_t D,
             int64_t E, int dtype, int act, void* stream);

/* Bytes of device workspace fmlp_fwd_ws can use for these shapes and dtype on the current
 * device (0 when the forward needs none). No counterpart in the reference. */
size_t fmlp_fwd_workspace_bytes(int64_t H, int64_t B, int64_t D, int64_t E, int dtype);

/* fmlp_fwd with a device workspace (16-byte aligned, or NULL). No counterpart in the reference,
 * whose forward allocates only o: with at least fmlp_fwd_workspace_bytes() bytes, a grid whose
 * last round of tiles would leave most CUs idle (a short last round after full ones, e.g. a
 * ragged B just past a multiple of the CU count) splits those tiles over E across workgroups.
 * The parts' fp32 partials go through the workspace and a second launch sums them in a fixed
 * order. With a smaller workspace or NULL it is fmlp_fwd. The workspace is scratch for the
 * duration of the call on `stream`. */
int fmlp_fwd_ws(const void* x, const void* w1, const void* w2, void* o, int64_t H, int64_t B, int64_t D,
                int64_t E, int dtype, int act, void* workspace, size_t workspace_bytes, void* stream);

/* fmlp_fwd with X (H,B,D), W1 (H,D,E), W2 (H,E,D) given as strided views: each *_strides is
 * three non-negative element strides (head, row, column); o stays dense. No counterpart in
 * the reference, whose wrapper copies such views through reshape / contiguous
 * (flashmlp.py:453-459): for callers holding sliced or transposed tensors. Dense strides
 * take the tuned kernels when the shape allows, other strides the generic kernels. */
int fmlp_fwd_strided(const void* x, const void* w1, const void* w2, void* o, int64_t H, int64_t B, int64_t D,
                     int64_t E, const int64_t* x_strides, const int64_t* w1_strides, const int64_t* w2_strides,
                     int dtype, int act, void* stream);

/* Bytes of device workspace fmlp_bwd / fmlp_bwd_strided need for these shapes and dtype flags
 * on the current device, whatever the activation (0 when none is needed). Every backward flag
 * can change it (FMLP_DW_HILO, FMLP_BWD_RECOMPUTE and FMLP_BWD_STORE_DZ change the plan,
 * FMLP_BWD_NO_DX leaves only the dW programs' partials, FMLP_BWD_NO_DW only the split ragged dX
 * tiles' partials, 0 where the plan splits none): query it with the flags of the call it is for. For
 * shapes the tuned kernels do not take, it is the fp32 partials of the generic dW programs'
 * B split (16-bit D = 256 with E % 8 == 0: the larger of that and the D = 256 dW programs'
 * split); those calls (and fmlp_bwd_strided calls whose views send a tuned shape to the
 * generic kernels) accept any workspace, NULL included, and split B only as far as it fits. */
size_t fmlp_bwd_workspace_bytes(int64_t H, int64_t B, int64_t D, int64_t E, int dtype);

/* 1 when fmlp_bwd takes the stored-dZ form for these shapes, dtype flags and activation on the
 * current device, else 0 (also for rejected arguments and for a partial backward,
 * FMLP_BWD_NO_DX or FMLP_BWD_NO_DW, which stores none). No counterpart in the reference: for
 * callers planning memory and for benches naming the kernels they time. */
int fmlp_bwd_stores_dz(int64_t H, int64_t B, int64_t D, int64_t E, int dtype, int act);

/* The tuned backward's plan for these shapes, dtype flags and activation on the current
 * device, written to info[0 .. n_info - 1] (at most 11 values, in this order): stored-dZ form
 * (0/1), B splits of the dW programs, dX programs' in-workgroup E parts, parts of each split
 * ragged dX tile (0: not split), dX programs first (0/1), dW programs, whole-tile dX programs,
 * split-tile dX programs, workspace bytes, the activation's code, and the E-columns per dW
 * program (128 or 64). With FMLP_BWD_NO_DX or FMLP_BWD_NO_DW it describes what such a call
 * launches (the dW programs alone, or the dX programs alone over whole tiles) and the workspace
 * it needs. Also for dense 16-bit D = 256 with E % 8 == 0 (the D = 256 dX and dW
 * programs, one launch each; the split as with an unlimited workspace, which such calls take
 * only as far as their workspace holds). Returns FMLP_OK, or FMLP_ERR_UNSUPPORTED for shapes
 * the generic kernels take. No counterpart in the reference: a diagnostic for tests and
 * benches. */
int fmlp_bwd_plan(int64_t H, int64_t B, int64_t D, int64_t E, int dtype, int act, int64_t* info, int n_info);

/*
 * Backward: dx = dZ @ w1^T, dw1 = x^T @ dZ, dw2 = h^T @ dout with h = act(x @ w1),
 * dZ = (dout @ w2^T) * act'(x @ w1); Z and h are recomputed from x, never stored by the forward.
 * Replaces flashmlp_bwd's kernel launch (flashmlp.py:480-538, kernel flashmlp.py:341-421).
 * Two forms, chosen per shape by an estimate of their time: the reference's, whose dX programs
 * recompute Z and dH (one launch), and a stored-dZ form for large shapes, whose dW programs
 * also write dZ (in the io dtype: the value the dX product takes) to the workspace and dx is a
 * GEMM over it (two launches, 10u instead of 14u of matrix work, u = H B D E, at
 * H ceil(E/128) 128 ceil(B/256) 256 io elements of workspace). FMLP_BWD_RECOMPUTE keeps the
 * first. dx, dw1, dw2 are fully overwritten. `workspace` may be NULL when
 * fmlp_bwd_workspace_bytes() is 0.
 */
int fmlp_bwd(const void* x, const void* w1, const void* w2, const void* dout, void* dx, void* dw1, void* dw2,
             int64_t H, int64_t B, int64_t D, int64_t E, int dtype, int act, void* workspace,
             size_t workspace_bytes, void* stream);

/* fmlp_bwd with X, W1, W2 and dout given as strided views (three element strides each, as in
 * fmlp_fwd_strided); dx, dw1, dw2 stay dense. No counterpart in the reference (its wrapper
 * copies dout with .contiguous(), flashmlp.py:508). The workspace rule is fmlp_bwd's. */
int fmlp_bwd_strided(const void* x, const void* w1, const void* w2, const void* dout, void* dx, void* dw1,
                     void* dw2, int64_t H, int64_t B, int64_t D, int64_t E, const int64_t* x_strides,
                     const int64_t* w1_strides, const int64_t* w2_strides, const int64_t* dout_strides, int dtype,
                     int act, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Backward without allocation: fmlp_bwd with the workspace replaced by the library's own
 * static device scratch (FMLP_SCRATCH_MAX_BYTES per device, in a code object of its own that is
 * loaded onto a device, and so reserved there, at the first fmlp_bwd_noalloc call on it, until
 * the process ends; processes that never call it do not hold it). No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). It calls no hipMalloc, hipFree or
 * allocating routine. Its plan only considers B splits of the dW programs, and the stored-dZ
 * form, whose workspace fits the scratch: where fmlp_bwd would split B more finely (or store
 * dZ) than the scratch allows, it takes a smaller split (or the recompute form) instead of
 * failing, so its dW results can differ from fmlp_bwd's in the last bits (summation order)
 * and it is never FMLP_ERR_WORKSPACE. All calls on one device share that device's scratch:
 * calls that overlap on one device (other streams, other threads) race; serialise them.
 */
#define FMLP_SCRATCH_MAX_BYTES ((size_t)64 << 20)
int fmlp_bwd_noalloc(const void* x, const void* w1, const void* w2, const void* dout, void* dx, void* dw1, void* dw2,
                     int64_t H, int64_t B, int64_t D, int64_t E, int dtype, int act, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FLASHMLP_H_ */
