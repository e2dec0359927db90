// Generic FlashMLP kernels for gfx950: the shapes and layouts the tuned kernels
// (fmlp_fwd.hip, fmlp_bwd.hip) do not take.
//
//   * D in {16, 32, 64, 128, 256} (the reference's D is a power of two >= 16: tl.arange(0, D),
//     flashmlp.py:66,186), any E >= 1, any B;
//   * io dtype fp16, bf16 or fp32 (the reference's io dtype is x's, flashmlp.py:87,183,265,367);
//     16-bit io uses v_mfma_f32_32x32x16_{f16,bf16}, fp32 io v_mfma_f32_32x32x2_f32;
//   * inputs X, W1, W2, dO with arbitrary element strides (views, no copies); outputs are
//     dense row-major.
// Same algorithm and cast points as the tuned kernels: fp32 accumulation, h rounded to the io
// dtype before O += h W2 (flashmlp.py:141-147), dZ and h rounded before the dX / dW products
// (flashmlp.py:215-235,297-320) -- no rounding at all for fp32 io -- Z and h recomputed in the
// backward, Leaky ReLU's derivative at Z == 0 from autograd (0.01).
//
// Operands are read straight from global memory (L1/L2 cached) per MFMA: simple and
// stride-agnostic, not tuned. One wave per SIMD (four waves per workgroup), so a wave may
// hold the D = 256 accumulators.
//
// MFMA 32x32 C layout (both instructions): lane l holds column n = l % 32 and rows
// m = 8 (i / 4) + 4 (l / 32) + i % 4 for i = 0..15. A K = 16 operand holds k-slots 8 (l / 32)
// + j, j < 8; a K = 2 operand holds k-slot l / 32.
#include "fmlp_device.h"
#include "fmlp_launch.h"

#include <type_traits>

namespace fmlp {

namespace {

template <int IO>
struct Gen {
  static constexpr bool W16 = IO != IO_F32;
  static constexpr bool BF = IO == IO_BF16;
  static constexpr int K = W16 ? 16 : 2;  // k per MFMA
};

// raw 16-bit element / fp32 element at an element index
__device__ __forceinline__ unsigned ld16(const void* p, long long i) { return ((const u16*)p)[i]; }
__device__ __forceinline__ float ld32(const void* p, long long i) { return ((const float*)p)[i]; }

template <int IO>
__device__ __forceinline__ float ld_f(const void* p, long long i) {
  if constexpr (IO == IO_F32) return ld32(p, i);
  else return to_f32<IO == IO_BF16>((u16)ld16(p, i));
}

// 16-bit operand: slot j = element f(j) (raw bits), j = 0..7; zeros when !ok
template <typename F>
__device__ __forceinline__ u32x4 op16(bool ok, F f) {
  u32x4 r = {0u, 0u, 0u, 0u};
  if (ok) {
#pragma unroll
    for (int w = 0; w < 4; ++w) r[w] = f(2 * w) | (f(2 * w + 1) << 16);
  }
  return r;
}

__device__ __forceinline__ f32x16 mma16(bool bf, const u32x4& a, const u32x4& b, const f32x16& c) {
  return bf ? mfma<true>(a, b, c) : mfma<false>(a, b, c);
}
__device__ __forceinline__ f32x16 mma32(float a, float b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// activation selected at run time (a wave-uniform kernel argument)
__device__ __forceinline__ float act_rt(int act, float z) {
  switch (act) {
    case ACT_SILU: return act_f<ACT_SILU>(z);
    case ACT_LEAKY: return act_f<ACT_LEAKY>(z);
    case ACT_SIGMOID: return act_f<ACT_SIGMOID>(z);
    default: return z;
  }
}
__device__ __forceinline__ void act_fb_rt(int act, float z, float dh, float& h, float& dz) {
  switch (act) {
    case ACT_SILU: act_fb<ACT_SILU>(z, dh, h, dz); break;
    case ACT_LEAKY: act_fb<ACT_LEAKY>(z, dh, h, dz); break;
    case ACT_SIGMOID: act_fb<ACT_SIGMOID>(z, dh, h, dz); break;
    default: h = z; dz = dh;
  }
}

// value rounded to the io dtype (no-op for fp32 io)
template <int IO>
__device__ __forceinline__ float io_round(float v) {
  if constexpr (IO == IO_F32) return v;
  else return lo_f32<IO == IO_BF16>(pack2<IO == IO_BF16>(v, 0.f));
}
template <int IO>
__device__ __forceinline__ unsigned io_bits(float v) {  // 16-bit io only
  return pack2<IO == IO_BF16>(v, 0.f) & 0xffffu;
}

// store one output element (dense row-major), io dtype or fp32 (outf32)
template <int IO>
__device__ __forceinline__ void st_out(void* p, long long i, float v, int outf32) {
  if (outf32 || IO == IO_F32) ((float*)p)[i] = v;
  else ((u16*)p)[i] = (u16)io_bits<IO>(v);
}

// a wave-uniform value the compiler must treat as unknown at this point: keeps address
// arithmetic inside the loop iteration instead of hoisting dozens of precomputed addresses
// into registers across the loop
__device__ __forceinline__ long long opaque(long long v) {
  asm volatile("" : "+s"(v));
  return v;
}

constexpr int GEN_NT = 256;  // four waves
constexpr int GEN_ROWS = 128;  // rows per forward / dX workgroup (32 per wave)
constexpr int GEN_COLS = 128;  // E columns per dW workgroup (32 per wave)

}  // namespace

// ------------------------------------------------------------------------------------
// Forward: wave = 32 rows b; per 32-column E-chunk, Z^T (lane = row) from W1c^T and X^T,
// h = act(Z^T) rounded to the io dtype, O += h W2c (lane = column d).
// ------------------------------------------------------------------------------------
template <int IO, int D>
__global__ void __launch_bounds__(GEN_NT) __attribute__((amdgpu_waves_per_eu(1, 1)))
gen_fwd_kernel(GenArgs a, int tiles_per_head) {
  using G = Gen<IO>;
  constexpr int K = G::K, KS = D / K, NTN = (D + 31) / 32;
  using Op = typename std::conditional<G::W16, u32x4, float>::type;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 5, l32 = lane & 31;
  const int h = blockIdx.x / tiles_per_head, bt = blockIdx.x % tiles_per_head;
  const int b0 = bt * GEN_ROWS + wave * 32;
  const long long B = a.B, E = a.E;
  const long long xb = h * a.sx[0], w1b = h * a.sw1[0], w2b = h * a.sw2[0];

  // X^T operand: lane = row b0 + l32, k-slots d (read per chunk; L1 / L2 serve the repeats)
  const int bx = b0 + l32;
  const long long rb = xb + (long long)bx * a.sx[1];
  auto xop = [&](int ks, long long sx2) -> Op {
    if constexpr (G::W16) return op16(bx < B, [&](int j) { return ld16(a.x, rb + (long long)(ks * 16 + 8 * g + j) * sx2); });
    else return bx < B ? ld32(a.x, rb + (long long)(2 * ks + g) * sx2) : 0.f;
  };
  f32x16 o[NTN];
#pragma unroll
  for (int nt = 0; nt < NTN; ++nt) o[nt] = zero16();

  for (long long c0 = 0; c0 < E; c0 += 32) {
    const long long sx2 = opaque(a.sx[2]), sw11 = opaque(a.sw1[1]), sw12 = opaque(a.sw1[2]);
    const long long sw21 = opaque(a.sw2[1]), sw22 = opaque(a.sw2[2]);
    // Z^T (M = e, N = b): A = W1c^T, lane = column e
    const long long e = c0 + l32;
    f32x16 z = zero16();
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if constexpr (G::W16) {
        const u32x4 A = op16(e < E, [&](int j) { return ld16(a.w1, w1b + (long long)(ks * 16 + 8 * g + j) * sw11 + e * sw12); });
        z = mma16(G::BF, A, xop(ks, sx2), z);
      } else {
        const float A = e < E ? ld32(a.w1, w1b + (long long)(2 * ks + g) * sw11 + e * sw12) : 0.f;
        z = mma32(A, xop(ks, sx2), z);
      }
      asm volatile("" ::: "memory");  // loads stay in their step (bounded live ranges)
    }
    // h: lane = row b0 + l32, value i = column e_i = c0 + 8 (i / 4) + 4 g + i % 4
    float hv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) hv[i] = io_round<IO>(act_rt(a.act, z[i]));
    // O += h W2c: B = W2c, lane = column d, k-slots e (in h's order); rows e past E read 0
#pragma unroll
    for (int nt = 0; nt < NTN; ++nt) {
      const int d = nt * 32 + l32;
      if constexpr (G::W16) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          u32x4 A;
#pragma unroll
          for (int w = 0; w < 4; ++w) A[w] = pack2<G::BF>(hv[8 * s + 2 * w], hv[8 * s + 2 * w + 1]);
          const u32x4 Bv = op16(d < D, [&](int j) {
            const long long ee = c0 + 16 * s + 8 * (j / 4) + 4 * g + (j & 3);
            return ee < E ? ld16(a.w2, w2b + ee * sw21 + (long long)d * sw22) : 0u;
          });
          o[nt] = mma16(G::BF, A, Bv, o[nt]);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const long long ee = c0 + 8 * (i / 4) + 4 * g + (i & 3);
          const float Bv = (d < D && ee < E) ? ld32(a.w2, w2b + ee * sw21 + (long long)d * sw22) : 0.f;
          o[nt] = mma32(hv[i], Bv, o[nt]);
        }
      }
      asm volatile("" ::: "memory");
    }
  }
  // O (M = b, N = d): lane = column d, value i = row b0 + 8 (i / 4) + 4 g + i % 4
#pragma unroll
  for (int nt = 0; nt < NTN; ++nt) {
    const int d = nt * 32 + l32;
    if (d < D) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const long long b = b0 + 8 * (i / 4) + 4 * g + (i & 3);
        if (b < B) st_out<IO>(a.o, ((long long)h * B + b) * D + d, o[nt][i], a.out_f32);
      }
    }
  }
}

// ------------------------------------------------------------------------------------
// dX: wave = 32 rows; per E-chunk Z^T and dH^T = W2c dO^T (lane = row), dZ = dH act'(Z)
// rounded to the io dtype, dX += dZ W1c^T (lane = column d).
// ------------------------------------------------------------------------------------
template <int IO, int D>
__global__ void __launch_bounds__(GEN_NT) __attribute__((amdgpu_waves_per_eu(1, 1)))
gen_dx_kernel(GenArgs a, int tiles_per_head) {
  using G = Gen<IO>;
  constexpr int K = G::K, KS = D / K, NTN = (D + 31) / 32;
  using Op = typename std::conditional<G::W16, u32x4, float>::type;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 5, l32 = lane & 31;
  const int h = blockIdx.x / tiles_per_head, bt = blockIdx.x % tiles_per_head;
  const int b0 = bt * GEN_ROWS + wave * 32;
  const long long B = a.B, E = a.E;
  const long long xb = h * a.sx[0], db = h * a.sdo[0], w1b = h * a.sw1[0], w2b = h * a.sw2[0];

  // X^T / dO^T operands: lane = row b0 + l32, k-slots d (read per chunk)
  const int bx = b0 + l32;
  const long long rx = xb + (long long)bx * a.sx[1], rd = db + (long long)bx * a.sdo[1];
  auto rop = [&](const void* p, long long rbase, long long sd, int ks) -> Op {  // sd: the column stride
    if constexpr (G::W16) return op16(bx < B, [&](int j) { return ld16(p, rbase + (long long)(ks * 16 + 8 * g + j) * sd); });
    else return bx < B ? ld32(p, rbase + (long long)(2 * ks + g) * sd) : 0.f;
  };
  f32x16 acc[NTN];
#pragma unroll
  for (int nt = 0; nt < NTN; ++nt) acc[nt] = zero16();

  for (long long c0 = 0; c0 < E; c0 += 32) {
    const long long sx2 = opaque(a.sx[2]), sdo2 = opaque(a.sdo[2]), sw11 = opaque(a.sw1[1]), sw12 = opaque(a.sw1[2]);
    const long long sw21 = opaque(a.sw2[1]), sw22 = opaque(a.sw2[2]);
    const long long e = c0 + l32;
    f32x16 z = zero16(), dh = zero16();
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if constexpr (G::W16) {
        const u32x4 A1 = op16(e < E, [&](int j) { return ld16(a.w1, w1b + (long long)(ks * 16 + 8 * g + j) * sw11 + e * sw12); });
        const u32x4 A2 = op16(e < E, [&](int j) { return ld16(a.w2, w2b + e * sw21 + (long long)(ks * 16 + 8 * g + j) * sw22); });
        z = mma16(G::BF, A1, rop(a.x, rx, sx2, ks), z);
        dh = mma16(G::BF, A2, rop(a.dout, rd, sdo2, ks), dh);
      } else {
        const float A1 = e < E ? ld32(a.w1, w1b + (long long)(2 * ks + g) * sw11 + e * sw12) : 0.f;
        const float A2 = e < E ? ld32(a.w2, w2b + e * sw21 + (long long)(2 * ks + g) * sw22) : 0.f;
        z = mma32(A1, rop(a.x, rx, sx2, ks), z);
        dh = mma32(A2, rop(a.dout, rd, sdo2, ks), dh);
      }
      asm volatile("" ::: "memory");
    }
    float dz[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float hh, dd;
      act_fb_rt(a.act, z[i], dh[i], hh, dd);
      dz[i] = io_round<IO>(dd);
    }
    // dX += dZ W1c^T: B = W1c^T, lane = column d, k-slots e (in dZ's order)
#pragma unroll
    for (int nt = 0; nt < NTN; ++nt) {
      const int d = nt * 32 + l32;
      if constexpr (G::W16) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          u32x4 A;
#pragma unroll
          for (int w = 0; w < 4; ++w) A[w] = pack2<G::BF>(dz[8 * s + 2 * w], dz[8 * s + 2 * w + 1]);
          const u32x4 Bv = op16(d < D, [&](int j) {
            const long long ee = c0 + 16 * s + 8 * (j / 4) + 4 * g + (j & 3);
            return ee < E ? ld16(a.w1, w1b + (long long)d * sw11 + ee * sw12) : 0u;
          });
          acc[nt] = mma16(G::BF, A, Bv, acc[nt]);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const long long ee = c0 + 8 * (i / 4) + 4 * g + (i & 3);
          const float Bv = (d < D && ee < E) ? ld32(a.w1, w1b + (long long)d * sw11 + ee * sw12) : 0.f;
          acc[nt] = mma32(dz[i], Bv, acc[nt]);
        }
      }
      asm volatile("" ::: "memory");
    }
  }
#pragma unroll
  for (int nt = 0; nt < NTN; ++nt) {
    const int d = nt * 32 + l32;
    if (d < D) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const long long b = b0 + 8 * (i / 4) + 4 * g + (i & 3);
        if (b < B) st_out<IO>(a.dx, ((long long)h * B + b) * D + d, acc[nt][i], a.out_f32);
      }
    }
  }
}

// ------------------------------------------------------------------------------------
// dW: wave = 32 E-columns of one head over every row, in 32-row subtiles: Z = X W1c and
// dH = dO W2c^T (lane = column e), h and dZ rounded to the io dtype, dW2 += h^T dO and
// dW1^T += dZ^T X (lane = column d, rows e).
// ------------------------------------------------------------------------------------
template <int IO, int D>
__global__ void __launch_bounds__(GEN_NT) __attribute__((amdgpu_waves_per_eu(1, 1)))
gen_dw_kernel(GenArgs a, int tiles_per_head) {
  using G = Gen<IO>;
  constexpr int KS = D / G::K, NTN = (D + 31) / 32;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 5, l32 = lane & 31;
  const int h = blockIdx.x / tiles_per_head, et = blockIdx.x % tiles_per_head;
  const long long e0 = (long long)et * GEN_COLS + wave * 32;
  const long long B = a.B, E = a.E;
  const long long xb = h * a.sx[0], db = h * a.sdo[0], w1b = h * a.sw1[0], w2b = h * a.sw2[0];
  const long long e = e0 + l32;  // this lane's column in Z / dH

  f32x16 a1[NTN], a2[NTN];  // dW1^T and dW2 (M = e, N = d)
#pragma unroll
  for (int nt = 0; nt < NTN; ++nt) {
    a1[nt] = zero16();
    a2[nt] = zero16();
  }
  for (long long r0 = 0; r0 < B; r0 += 32) {
    const long long sx1 = opaque(a.sx[1]), sx2 = opaque(a.sx[2]), sdo1 = opaque(a.sdo[1]), sdo2 = opaque(a.sdo[2]);
    const long long sw11 = opaque(a.sw1[1]), sw12 = opaque(a.sw1[2]), sw21 = opaque(a.sw2[1]), sw22 = opaque(a.sw2[2]);
    // Z, dH (M = rows, N = e): A = X / dO rows (lane = row r0 + l32), B = W1c / W2c^T (lane = e)
    const long long rA = r0 + l32;
    f32x16 z = zero16(), dh = zero16();
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if constexpr (G::W16) {
        const u32x4 Ax = op16(rA < B, [&](int j) { return ld16(a.x, xb + rA * sx1 + (long long)(ks * 16 + 8 * g + j) * sx2); });
        const u32x4 Ad = op16(rA < B, [&](int j) { return ld16(a.dout, db + rA * sdo1 + (long long)(ks * 16 + 8 * g + j) * sdo2); });
        const u32x4 B1 = op16(e < E, [&](int j) { return ld16(a.w1, w1b + (long long)(ks * 16 + 8 * g + j) * sw11 + e * sw12); });
        const u32x4 B2 = op16(e < E, [&](int j) { return ld16(a.w2, w2b + e * sw21 + (long long)(ks * 16 + 8 * g + j) * sw22); });
        z = mma16(G::BF, Ax, B1, z);
        dh = mma16(G::BF, Ad, B2, dh);
      } else {
        const long long d = 2 * ks + g;
        const float Ax = rA < B ? ld32(a.x, xb + rA * sx1 + d * sx2) : 0.f;
        const float Ad = rA < B ? ld32(a.dout, db + rA * sdo1 + d * sdo2) : 0.f;
        const float B1 = e < E ? ld32(a.w1, w1b + d * sw11 + e * sw12) : 0.f;
        const float B2 = e < E ? ld32(a.w2, w2b + e * sw21 + d * sw22) : 0.f;
        z = mma32(Ax, B1, z);
        dh = mma32(Ad, B2, dh);
      }
      asm volatile("" ::: "memory");
    }
    // h, dZ: lane = column e, value i = row r0 + 8 (i / 4) + 4 g + i % 4 (rows past B: X, dO
    // are zero there, so dZ = 0 and h multiplies a zero dO row)
    // (16-bit io rounds h and dZ when packing them into the operands below)
    float hv[16], dz[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) act_fb_rt(a.act, z[i], dh[i], hv[i], dz[i]);
    // dW2 += h^T dO, dW1^T += dZ^T X: A from h / dZ (lane = e), B = dO / X (lane = column d,
    // k-slots rows in h's order)
#pragma unroll
    for (int nt = 0; nt < NTN; ++nt) {
      const int d = nt * 32 + l32;
      if constexpr (G::W16) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          u32x4 Ah, Az, AhL, AzL;  // io-rounded terms, and the lo terms v - round(v) (hilo)
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const float h0 = hv[8 * s + 2 * w], h1 = hv[8 * s + 2 * w + 1];
            const float z0 = dz[8 * s + 2 * w], z1 = dz[8 * s + 2 * w + 1];
            Ah[w] = pack2<G::BF>(h0, h1);
            Az[w] = pack2<G::BF>(z0, z1);
            AhL[w] = pack2<G::BF>(h0 - lo_f32<G::BF>(Ah[w]), h1 - hi_f32<G::BF>(Ah[w]));
            AzL[w] = pack2<G::BF>(z0 - lo_f32<G::BF>(Az[w]), z1 - hi_f32<G::BF>(Az[w]));
          }
          auto row = [&](int j) { return r0 + 16 * s + 8 * (j / 4) + 4 * g + (j & 3); };
          const u32x4 Bd = op16(d < D, [&](int j) {
            const long long r = row(j);
            return r < B ? ld16(a.dout, db + r * sdo1 + (long long)d * sdo2) : 0u;
          });
          const u32x4 Bx = op16(d < D, [&](int j) {
            const long long r = row(j);
            return r < B ? ld16(a.x, xb + r * sx1 + (long long)d * sx2) : 0u;
          });
          a2[nt] = mma16(G::BF, Ah, Bd, a2[nt]);
          a1[nt] = mma16(G::BF, Az, Bx, a1[nt]);
          if (a.hilo) {
            a2[nt] = mma16(G::BF, AhL, Bd, a2[nt]);
            a1[nt] = mma16(G::BF, AzL, Bx, a1[nt]);
          }
          asm volatile("" ::: "memory");
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const long long r = r0 + 8 * (i / 4) + 4 * g + (i & 3);
          const bool ok = d < D && r < B;
          const float Bd = ok ? ld32(a.dout, db + r * sdo1 + (long long)d * sdo2) : 0.f;
          const float Bx = ok ? ld32(a.x, xb + r * sx1 + (long long)d * sx2) : 0.f;
          a2[nt] = mma32(hv[i], Bd, a2[nt]);
          a1[nt] = mma32(dz[i], Bx, a1[nt]);
        }
      }
      asm volatile("" ::: "memory");
    }
  }
  // dW2[h][e][d], dW1[h][d][e]: lane = column d, value i = row e0 + 8 (i / 4) + 4 g + i % 4
#pragma unroll
  for (int nt = 0; nt < NTN; ++nt) {
    const int d = nt * 32 + l32;
    if (d < D) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const long long ee = e0 + 8 * (i / 4) + 4 * g + (i & 3);
        if (ee < E) {
          st_out<IO>(a.dw2, ((long long)h * E + ee) * D + d, a2[nt][i], a.out_f32);
          st_out<IO>(a.dw1, ((long long)h * D + d) * E + ee, a1[nt][i], a.out_f32);
        }
      }
    }
  }
}

// ------------------------------------------------------------------------------------
// launchers
// ------------------------------------------------------------------------------------
namespace {

template <int IO, int D>
hipError_t gen_launch_fwd_t(const GenArgs& a, hipStream_t st) {
  const long long tph = (a.B + GEN_ROWS - 1) / GEN_ROWS;
  const long long grid = tph * a.H;
  if (grid <= 0) return hipSuccess;
  if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL((gen_fwd_kernel<IO, D>), dim3((unsigned)grid), dim3(GEN_NT), 0, st, a, (int)tph);
  return hipGetLastError();
}

template <int IO, int D>
hipError_t gen_launch_bwd_t(const GenArgs& a, hipStream_t st) {
  const long long tph = (a.B + GEN_ROWS - 1) / GEN_ROWS;
  const long long ctph = (a.E + GEN_COLS - 1) / GEN_COLS;
  if (tph * a.H > 0x7fffffffLL || ctph * a.H > 0x7fffffffLL) return hipErrorInvalidValue;
  if (a.H > 0 && ctph > 0 && a.want_dw) {
    hipLaunchKernelGGL((gen_dw_kernel<IO, D>), dim3((unsigned)(ctph * a.H)), dim3(GEN_NT), 0, st, a, (int)ctph);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (a.H > 0 && tph > 0 && a.want_dx) {
    hipLaunchKernelGGL((gen_dx_kernel<IO, D>), dim3((unsigned)(tph * a.H)), dim3(GEN_NT), 0, st, a, (int)tph);
    return hipGetLastError();
  }
  return hipSuccess;
}

template <int IO>
hipError_t gen_dispatch(const GenArgs& a, hipStream_t st, bool fwd) {
  switch (a.D) {
    case 16: return fwd ? gen_launch_fwd_t<IO, 16>(a, st) : gen_launch_bwd_t<IO, 16>(a, st);
    case 32: return fwd ? gen_launch_fwd_t<IO, 32>(a, st) : gen_launch_bwd_t<IO, 32>(a, st);
    case 64: return fwd ? gen_launch_fwd_t<IO, 64>(a, st) : gen_launch_bwd_t<IO, 64>(a, st);
    case 128: return fwd ? gen_launch_fwd_t<IO, 128>(a, st) : gen_launch_bwd_t<IO, 128>(a, st);
    case 256: return fwd ? gen_launch_fwd_t<IO, 256>(a, st) : gen_launch_bwd_t<IO, 256>(a, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t gen_run(const GenArgs& a, hipStream_t st, bool fwd) {
  switch (a.io) {
    case IO_F16: return gen_dispatch<IO_F16>(a, st, fwd);
    case IO_BF16: return gen_dispatch<IO_BF16>(a, st, fwd);
    case IO_F32: return gen_dispatch<IO_F32>(a, st, fwd);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_gen_fwd(const GenArgs& a, hipStream_t st) { return gen_run(a, st, true); }
hipError_t launch_gen_bwd(const GenArgs& a, hipStream_t st) { return gen_run(a, st, false); }

bool gen_supports_d(int64_t D) { return D == 16 || D == 32 || D == 64 || D == 128 || D == 256; }

}  // namespace fmlp
