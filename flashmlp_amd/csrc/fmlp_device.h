// Device-side building blocks shared by the FlashMLP gfx950 kernels.
//
// Conventions (all kernels):
//   * io element type is 16-bit (fp16 or bf16) held as `u16` in memory;
//   * every dense contraction is a v_mfma_f32_32x32x16_{bf16,f16} with fp32 accumulation;
//   * MFMA 32x32x16 lane layout (verified on MI355X):
//       A (M x K): lane l holds row m = l%32, k-slots 8*(l/32) + j, j = 0..7
//       B (K x N): lane l holds col n = l%32, k-slots 8*(l/32) + j
//       C (M x N): lane l holds col n = l%32, rows m = 8*(i/4) + 4*(l/32) + (i%4), i = 0..15
//     Only the pairing of A and B k-slots matters (a contraction is order free), so an
//     operand built from a C tile keeps the C row order as its k order and the other
//     operand is read with the same permutation.
//   * ds_read_b64_tr_b16 (verified): within each 16-lane group, lane i receives element
//     (i % 4) of the 8 bytes read by lanes 4*j + i/4, j = 0..3. Reading a 4x16 block of a
//     row-major 16-bit matrix (lane i reads row i/4, columns 4*(i%4)..+3) therefore gives
//     lane i column i, rows 0..3: a K-contiguous operand from an N-contiguous layout.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fmlp {

typedef unsigned short u16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

#define FMLP_LDS __attribute__((address_space(3)))

enum Act { ACT_NONE = 0, ACT_SILU = 1, ACT_LEAKY = 2, ACT_SIGMOID = 3 };

// 8 x 16-bit operand held as four dwords.
struct Frag { u32x4 v; };

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

template <bool BF16>
__device__ __forceinline__ f32x16 mfma(const u32x4& a, const u32x4& b, const f32x16& c) {
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

// Round-to-nearest-even conversion of two fp32 values into one dword of 16-bit values
// (low half = a). Lowers to v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32 on gfx950.
template <bool BF16>
__device__ __forceinline__ unsigned pack2(float a, float b) {
  if constexpr (BF16) {
    bf16x2 v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(unsigned, v);
  } else {
    f16x2 v = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(unsigned, v);
  }
}

template <bool BF16>
__device__ __forceinline__ float to_f32(u16 h) {
  if constexpr (BF16) {
    return __uint_as_float(((unsigned)h) << 16);
  } else {
    return (float)__builtin_bit_cast(_Float16, h);
  }
}

// the two 16-bit values of a pack2 dword (low half = first argument), widened exactly
template <bool BF16>
__device__ __forceinline__ float lo_f32(unsigned v) {
  if constexpr (BF16) return __uint_as_float(v << 16);
  else return (float)__builtin_bit_cast(_Float16, (u16)(v & 0xffffu));
}
template <bool BF16>
__device__ __forceinline__ float hi_f32(unsigned v) {
  if constexpr (BF16) return __uint_as_float(v & 0xffff0000u);
  else return (float)__builtin_bit_cast(_Float16, (u16)(v >> 16));
}

template <bool BF16>
__device__ __forceinline__ u16 from_f32(float f) {
  return (u16)(pack2<BF16>(f, 0.f) & 0xffffu);
}

// ---------------------------------------------------------------------------------
// Activations. Follows flashmlp.py:27-46 (forward) and PyTorch autograd for the
// derivatives (flashmlp.py:671-686 is differentiated by autograd in the oracle):
//   leaky(z) = z > 0 ? z : 0.01 z        leaky'(z) = z > 0 ? 1 : 0.01   (autograd at z == 0)
//   silu(z)  = z * s(z)                  silu'(z) = s + h (1 - s), h = z s (fp32)
//   sigmoid(z) = s(z)                    sigmoid'(z) = s (1 - s)
// s(z) = 1 / (1 + 2^(-z * log2 e)) : the definition of the logistic function with
// e^x = 2^(x log2 e); v_exp_f32 and v_rcp_f32 are the hardware base-2 exponential and
// reciprocal (each accurate to about 1 ulp).
// ---------------------------------------------------------------------------------
__device__ __forceinline__ float sigm(float z) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(z * -1.4426950408889634f));
}

template <int ACT>
__device__ __forceinline__ float act_f(float z) {
  if constexpr (ACT == ACT_SILU) return z * sigm(z);
  else if constexpr (ACT == ACT_LEAKY) return z > 0.f ? z : 0.01f * z;
  else if constexpr (ACT == ACT_SIGMOID) return sigm(z);
  else return z;
}

// h = act(z) and dz = dh * act'(z)
template <int ACT>
__device__ __forceinline__ void act_fb(float z, float dh, float& h, float& dz) {
  if constexpr (ACT == ACT_SILU) {
    float s = sigm(z);
    h = z * s;
    dz = dh * __builtin_fmaf(h, 1.0f - s, s);
  } else if constexpr (ACT == ACT_LEAKY) {
    bool p = z > 0.f;
    h = p ? z : 0.01f * z;
    dz = p ? dh : 0.01f * dh;
  } else if constexpr (ACT == ACT_SIGMOID) {
    float s = sigm(z);
    h = s;
    dz = dh * (s - s * s);
  } else {
    h = z;
    dz = dh;
  }
}

// dz only (dX programs never need h)
template <int ACT>
__device__ __forceinline__ float act_b(float z, float dh) {
  if constexpr (ACT == ACT_SILU) {
    float s = sigm(z);
    float h = z * s;
    return dh * __builtin_fmaf(h, 1.0f - s, s);
  } else if constexpr (ACT == ACT_LEAKY) {
    return z > 0.f ? dh : 0.01f * dh;
  } else if constexpr (ACT == ACT_SIGMOID) {
    float s = sigm(z);
    return dh * (s - s * s);
  } else {
    return dh;
  }
}

// ---------------------------------------------------------------------------------
// LDS access helpers. Kernels use dynamic shared memory only, addressed by byte offset
// from its start. Offsets are signed and applied as in-bounds pointer arithmetic, which
// lets the compiler move constant parts into the DS instructions' immediate offset field.
// ---------------------------------------------------------------------------------
extern __shared__ __attribute__((aligned(16))) char fmlp_lds[];

__device__ __forceinline__ u32x4 lds_read16(int byte_off) {
  return *(const FMLP_LDS u32x4*)((FMLP_LDS char*)fmlp_lds + byte_off);
}
__device__ __forceinline__ u32x2 lds_read8(int byte_off) {
  return *(const FMLP_LDS u32x2*)((FMLP_LDS char*)fmlp_lds + byte_off);
}
__device__ __forceinline__ u32x2 lds_read_tr(int byte_off) {
  i16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((FMLP_LDS i16x4*)((FMLP_LDS char*)fmlp_lds + byte_off));
  return __builtin_bit_cast(u32x2, r);
}
__device__ __forceinline__ void lds_write16(int byte_off, const u32x4& v) {
  *(FMLP_LDS u32x4*)((FMLP_LDS char*)fmlp_lds + byte_off) = v;
}
__device__ __forceinline__ void lds_write8(int byte_off, const u32x2& v) {
  *(FMLP_LDS u32x2*)((FMLP_LDS char*)fmlp_lds + byte_off) = v;
}
__device__ __forceinline__ u32x4 cat(const u32x2& lo, const u32x2& hi) {
  u32x4 r = {lo[0], lo[1], hi[0], hi[1]};
  return r;
}

// ---------------------------------------------------------------------------------
// Raw buffer loads (stride-0 buffer resource). A load at a byte offset at or beyond the
// resource's size returns zeros without touching memory, so the edge tiles of a loop need
// no branches: the loop body stays one basic block and the compiler keeps the
// instruction order the step schedules ask for. Word 3 0x00020000 is the gfx9-family
// resource format (32-bit data format, no swizzle, no index stride).
// ---------------------------------------------------------------------------------
typedef __amdgpu_buffer_rsrc_t Rsrc;
constexpr unsigned BUF_OOB = 0x80000000u;  // an offset beyond every resource make_rsrc builds

// `bytes` must be wave-uniform and in [0, 2^31); readfirstlane keeps the resource in scalar
// registers.
__device__ __forceinline__ Rsrc make_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, __builtin_amdgcn_readfirstlane(bytes),
                                           0x00020000);
}
// min(max(v, 0), hi) for wave-uniform v and hi. The readfirstlane between the two selects
// keeps the compiler from fusing them into a vector v_med3 (plus a readfirstlane back): the
// clamp stays two scalar instructions, off the VALU that the kernel loops are bound by.
__device__ __forceinline__ int clamp0(int v, int hi) {
  const int t = __builtin_amdgcn_readfirstlane(v < 0 ? 0 : v);
  return __builtin_amdgcn_readfirstlane(t > hi ? hi : t);
}
// Store of a wave's 32-row output tile in the MFMA C layout (lane = column 32 nt + l32 of a
// [rows][D] row-major tensor, rows b0 + 8 (i / 4) + 4 g + (i % 4) in acc[nt][i]), as the io
// dtype or, with outf32, as the fp32 sums. b0 is wave-uniform: the wave's rows get a buffer
// resource of their own, so rows at or past B fall outside it (no branches), and each
// store's offset is one of four lane registers (one per 8-row group) plus a constant in the
// instruction's offset field (at most (3 D + 96) 4 bytes < 4096).
template <bool BF16, int D>
__device__ __forceinline__ void store_rows(const f32x16 (&acc)[D / 32], void* __restrict__ out, size_t head_off, int B,
                                           int b0, int g, int l32, int outf32) {
  constexpr int NTN = D / 32;
  static_assert((3 * D + 96) * 4 < 4096, "store offsets within the immediate field");
  const int rows = clamp0(B - b0, 32);
  const int es = outf32 ? 4 : 2;
  const Rsrc r = make_rsrc((const char*)out + (head_off + (size_t)b0 * D) * es, rows * D * es);
  unsigned vo[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) vo[q] = (unsigned)((8 * q + 4 * g) * D + l32) * (unsigned)es;
  if (outf32) {
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
      for (int nt = 0; nt < NTN; ++nt)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[nt][i]), r,
                                              (int)(vo[i >> 2] + (unsigned)(((i & 3) * D + nt * 32) * 4)), 0, 0);
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
      for (int nt = 0; nt < NTN; ++nt)
        __builtin_amdgcn_raw_buffer_store_b16(from_f32<BF16>(acc[nt][i]), r,
                                              (int)(vo[i >> 2] + (unsigned)(((i & 3) * D + nt * 32) * 2)), 0, 0);
  }
}
__device__ __forceinline__ u32x4 buf_load16(Rsrc r, unsigned byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, 0);
}

// 16 bytes per lane from a buffer straight into LDS (no registers): lane L's bytes land at
// lds_byte_off + 16 L (lds_byte_off wave-uniform; verified on MI355X). Issued as inline
// assembly on purpose: the compiler would otherwise treat every later LDS read as
// possibly reading the in-flight DMA data and wait for all of it, which removes the
// lookahead. Callers order DMA and reads themselves with wait_vmcnt<N>() (at most N
// vector-memory operations of the wave outstanding) and a workgroup barrier. Loads
// complete in issue order, so the compiler's own vmcnt waits stay correct (they can only
// become stricter). The resource words are those of make_rsrc (stride 0, gfx9 format).
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x4 make_rsrc_words(const void* base, int bytes) {
  const unsigned long long a = (unsigned long long)base;
  i32x4 w = {__builtin_amdgcn_readfirstlane((int)(unsigned)a), __builtin_amdgcn_readfirstlane((int)((a >> 32) & 0xffffu)),
             __builtin_amdgcn_readfirstlane(bytes), 0x00020000};
  return w;
}
__device__ __forceinline__ void buf_load16_lds(const i32x4& rsrc, unsigned byte_off, int lds_byte_off) {
  const unsigned m0 = (unsigned)__builtin_amdgcn_readfirstlane(
      (int)(unsigned)(uintptr_t)((FMLP_LDS char*)fmlp_lds + lds_byte_off));
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(byte_off), "s"(rsrc), "s"(m0)
               : "memory", "m0");
}
// The same with the non-temporal cache policy, for data a kernel reads exactly once and nothing
// reads after it (the stored dZ): its lines are not kept in the caches, so they do not evict
// what other streams still use.
__device__ __forceinline__ void buf_load16_lds_nt(const i32x4& rsrc, unsigned byte_off, int lds_byte_off) {
  const unsigned m0 = (unsigned)__builtin_amdgcn_readfirstlane(
      (int)(unsigned)(uintptr_t)((FMLP_LDS char*)fmlp_lds + lds_byte_off));
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen nt lds"
               :
               : "v"(byte_off), "s"(rsrc), "s"(m0)
               : "memory", "m0");
}
// cache-policy operand of the buffer store builtins: non-temporal (data written once, read once
// by a later kernel)
constexpr int CPOL_NT = 2;

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

// Row swizzle for row-major tiles whose rows are D 16-bit values (D = 64 or 128) and that
// are read both row-wise (16-byte chunks, lane m reads row m) and with ds_read_b64_tr_b16
// over 4-row x 32-byte blocks. 16-byte chunk c of row r is stored at chunk c ^ swz(r).
// With 64 LDS banks x 4 B both patterns are conflict free (measured on MI355X).
template <int D>
__device__ __forceinline__ unsigned swz16(unsigned r) {
  if constexpr (D == 128) return ((r & 3u) << 2) | ((r >> 2) & 3u);
  else return (((r >> 1) & 1u) << 2) | ((r >> 2) & 3u);
}
// byte offset of (row r, column d) inside a [rows][D] tile with the 16-byte swizzle;
// d must be a multiple of 4 (8-byte granularity).
template <int D>
__device__ __forceinline__ unsigned tile_off(unsigned r, unsigned d) {
  unsigned c = d >> 3;
  return r * (D * 2) + ((c ^ swz16<D>(r)) << 4) + ((d & 4u) << 1);
}

// W1 chunk tile [D rows][32 columns] (64-byte rows), read with ds_read_b64_tr_b16 over
// 4 consecutive rows and with ds_read_b64 down 32 consecutive rows. 8-byte unit u of row r
// is stored at unit u ^ ((r >> 2) & 7): conflict free for both patterns.
__device__ __forceinline__ unsigned w1c_off(unsigned r, unsigned unit) {
  return r * 64u + ((unit ^ ((r >> 2) & 7u)) << 3);
}

// W2 chunk tile [32 rows][D] stored as D/32 blocks of [32 rows][32 columns] (64-byte rows),
// read row-wise (lane m reads row m, one 16-byte piece). 16-byte piece q of row r (q < D/8)
// lives in block q/4 at chunk (q%4) ^ ((r >> 2) & 3): conflict free for 16 consecutive rows.
__device__ __forceinline__ unsigned w2s_off(unsigned r, unsigned q) {
  return (q >> 2) * 2048u + r * 64u + (((q & 3u) ^ ((r >> 2) & 3u)) << 4);
}

// ---------------------------------------------------------------------------------
// Step schedules. An iteration issues n1 MFMAs of one group and n2 of another; step j
// issues exactly one of them, with the n2 group spread evenly (Bresenham) among the n1.
// With the loops fully unrolled these fold to constants.
// ---------------------------------------------------------------------------------
__device__ __forceinline__ constexpr int sched_g2_before(int j, int n1, int n2) { return (j * n2) / (n1 + n2); }
__device__ __forceinline__ constexpr bool sched_is_g2(int j, int n1, int n2) {
  return sched_g2_before(j + 1, n1, n2) != sched_g2_before(j, n1, n2);
}
__device__ __forceinline__ constexpr int sched_index(int j, int n1, int n2) {
  return sched_is_g2(j, n1, n2) ? sched_g2_before(j, n1, n2) : j - sched_g2_before(j, n1, n2);
}
// Element e of an iteration's n_elem activations is computed at step (e * nsteps) / n_elem,
// i.e. step j computes elements [sched_elem_begin(j), sched_elem_begin(j + 1)). Loops over
// a step's elements take these bounds so that the element index depends on the step: an
// activation that did not would be loop invariant in the (not yet unrolled) step loop and
// could be hoisted out of it, which collapses the interleave.
__device__ __forceinline__ constexpr int sched_elem_begin(int j, int nsteps, int n_elem) {
  return (j * n_elem + nsteps - 1) / nsteps;
}

// ---------------------------------------------------------------------------------
// Workgroup -> tile remap. Workgroups are dispatched round-robin over the 8 XCDs
// (each with its own L2); this gives every XCD a contiguous range of logical tiles, so
// tiles of the same head (which share weights / activations) run on the same L2.
// Bijective on [0, n).
// ---------------------------------------------------------------------------------
__device__ __forceinline__ int xcd_remap(int bid, int n) {
  const int q = n >> 3, r = n & 7;
  const int x = bid & 7, j = bid >> 3;
  return x * q + (x < r ? x : r) + j;
}

}  // namespace fmlp
