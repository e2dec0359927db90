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

// 16-bit operand whose 8 k-slots are the columns 16 ks + 8 g .. + 7 of one row (element index of
// its column 0 at `rbase`, column stride `sd`): one 16-byte load when the host vouched that such
// runs are aligned vectors (`vec`, wave-uniform), else eight element loads; zeros when !ok
__device__ __forceinline__ u32x4 row_op16(const void* p, long long rbase, long long sd, int ks, int g, bool ok,
                                          int vec) {
  if (vec) {
    u32x4 r = {0u, 0u, 0u, 0u};
    if (ok) r = *(const u32x4*)((const u16*)p + rbase + ks * 16 + 8 * g);
    return r;
  }
  return op16(ok, [&](int j) { return ld16(p, rbase + (long long)(ks * 16 + 8 * g + j) * sd); });
}

// E split inside a workgroup (forward and dX kernels, for grids that leave CUs idle): the four
// waves are rt = 4 / ep row tiles of 32 rows times ep E-parts, part p walking the E-chunks
// c = p, p + ep, ...; the parts' partial output tiles are added through LDS in part order
// (deterministic), and part 0 stores.
template <int NTN>
__device__ __forceinline__ void gen_sum_parts(f32x16 (&acc)[NTN], int ep, int part, int rtile, int rt, int lane) {
  if (ep <= 1) return;
  // slot of (part p >= 1, row tile): NTN x 16 floats per lane, lane-major in 16-byte pieces
  auto slot = [&](int p) { return ((p - 1) * rt + rtile) * (NTN * 4096); };
  if (part > 0) {
#pragma unroll
    for (int nt = 0; nt < NTN; ++nt)
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4)
        lds_write16(slot(part) + ((nt * 4 + i4) * 64 + lane) * 16,
                    u32x4{__float_as_uint(acc[nt][4 * i4]), __float_as_uint(acc[nt][4 * i4 + 1]),
                          __float_as_uint(acc[nt][4 * i4 + 2]), __float_as_uint(acc[nt][4 * i4 + 3])});
  }
  __syncthreads();
  if (part == 0) {
    for (int p = 1; p < ep; ++p)
#pragma unroll
      for (int nt = 0; nt < NTN; ++nt)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
          const u32x4 v = lds_read16(slot(p) + ((nt * 4 + i4) * 64 + lane) * 16);
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[nt][4 * i4 + j] += __uint_as_float(v[j]);
        }
  }
}

// n steps of use(q, fetch(q)) with each step's operands fetched two steps ahead (a three-entry
// ring); the compiler barrier after each step keeps the loads in that order, so their latency
// overlaps two steps of matrix work without every load of the loop being hoisted into registers
template <int N, typename T, typename F, typename U>
__device__ __forceinline__ void pipelined(F fetch, U use) {
  T ring[3];
  ring[0] = fetch(0);
  if constexpr (N > 1) ring[1] = fetch(1);
#pragma unroll
  for (int q = 0; q < N; ++q) {
    if (q + 2 < N) ring[(q + 2) % 3] = fetch(q + 2);
    use(q, ring[q % 3]);
    asm volatile("" ::: "memory");
  }
}
template <typename T>
struct Pair {
  T a, b;
};

constexpr int GEN_NT = 256;  // four waves
constexpr int GEN_ROWS = 128;  // rows per forward / dX workgroup (32 per wave)
constexpr int GEN_COLS = 128;  // E columns per dW workgroup (32 per wave)
// D halves per dW wave: at D = 256 the two dW accumulator sets of a full row (256 registers) do
// not fit next to the rest, so two waves share 32 E-columns, each accumulating half of D (both
// compute the same Z and dH); the workgroup then covers 64 E-columns
constexpr int gen_dw_dsplit(int D) { return D == 256 ? 2 : 1; }
constexpr int gen_dw_cols(int D) { return GEN_COLS / gen_dw_dsplit(D); }

}  // namespace

// ------------------------------------------------------------------------------------
// Forward: wave = 32 rows b; per 32-column E-chunk, Z^T (lane = row) from W1c^T and X^T,
// h = act(Z^T) rounded to the io dtype, O += h W2c (lane = column d).
// ------------------------------------------------------------------------------------
template <int IO, int D>
__global__ void __launch_bounds__(GEN_NT) __attribute__((amdgpu_waves_per_eu(1, 1)))
gen_fwd_kernel(GenArgs a, int tiles_per_head, int ep) {
  using G = Gen<IO>;
  constexpr int K = G::K, KS = D / K, NTN = (D + 31) / 32;
  using Op = typename std::conditional<G::W16, u32x4, float>::type;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 5, l32 = lane & 31;
  const int rt = 4 / ep, rtile = wave % rt, part = wave / rt;  // row tile, E part
  const int h = blockIdx.x / tiles_per_head, bt = blockIdx.x % tiles_per_head;
  const int b0 = bt * (32 * rt) + rtile * 32;
  const long long B = a.B, E = a.E;
  const long long xb = h * a.sx[0], w1b = h * a.sw1[0], w2b = h * a.sw2[0];

  // X^T operand, loaded once for the whole E loop: lane = row b0 + l32, k-slots d
  const int bx = b0 + l32;
  const long long rb = xb + (long long)bx * a.sx[1];
  Op xr[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    if constexpr (G::W16) xr[ks] = row_op16(a.x, rb, a.sx[2], ks, g, bx < B, a.vec_x);
    else xr[ks] = bx < B ? ld32(a.x, rb + (long long)(2 * ks + g) * a.sx[2]) : 0.f;
  }
  f32x16 o[NTN];
#pragma unroll
  for (int nt = 0; nt < NTN; ++nt) o[nt] = zero16();

  for (long long c0 = 32LL * part; c0 < E; c0 += 32LL * ep) {
    const long long sw11 = opaque(a.sw1[1]), sw12 = opaque(a.sw1[2]);
    const long long sw21 = opaque(a.sw2[1]), sw22 = opaque(a.sw2[2]);
    // Z^T (M = e, N = b): A = W1c^T, lane = column e
    const long long e = c0 + l32;
    f32x16 z = zero16();
    pipelined<KS, Op>(
        [&](int ks) -> Op {
          if constexpr (G::W16)
            return op16(e < E, [&](int j) { return ld16(a.w1, w1b + (long long)(ks * 16 + 8 * g + j) * sw11 + e * sw12); });
          else return e < E ? ld32(a.w1, w1b + (long long)(2 * ks + g) * sw11 + e * sw12) : 0.f;
        },
        [&](int ks, const Op& A) {
          if constexpr (G::W16) z = mma16(G::BF, A, xr[ks], z);
          else z = mma32(A, xr[ks], z);
        });
    // h: lane = row b0 + l32, value i = column e_i = c0 + 8 (i / 4) + 4 g + i % 4
    float hv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) hv[i] = io_round<IO>(act_rt(a.act, z[i]));
    // O += h W2c: B = W2c, lane = column d, k-slots e (in h's order); rows e past E read 0
    if constexpr (G::W16) {
      u32x4 hA[2];
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int w = 0; w < 4; ++w) hA[s][w] = pack2<G::BF>(hv[8 * s + 2 * w], hv[8 * s + 2 * w + 1]);
      pipelined<2 * NTN, u32x4>(
          [&](int q) {
            const int nt = q >> 1, s = q & 1, d = nt * 32 + l32;
            return op16(d < D, [&](int j) {
              const long long ee = c0 + 16 * s + 8 * (j / 4) + 4 * g + (j & 3);
              return ee < E ? ld16(a.w2, w2b + ee * sw21 + (long long)d * sw22) : 0u;
            });
          },
          [&](int q, const u32x4& Bv) { o[q >> 1] = mma16(G::BF, hA[q & 1], Bv, o[q >> 1]); });
    } else {
      pipelined<16 * NTN, float>(
          [&](int q) {
            const int nt = q >> 4, i = q & 15, d = nt * 32 + l32;
            const long long ee = c0 + 8 * (i / 4) + 4 * g + (i & 3);
            return (d < D && ee < E) ? ld32(a.w2, w2b + ee * sw21 + (long long)d * sw22) : 0.f;
          },
          [&](int q, const float& Bv) { o[q >> 4] = mma32(hv[q & 15], Bv, o[q >> 4]); });
    }
  }
  gen_sum_parts<NTN>(o, ep, part, rtile, rt, lane);
  if (part > 0) return;
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
gen_dx_kernel(GenArgs a, int tiles_per_head, int ep) {
  using G = Gen<IO>;
  constexpr int K = G::K, KS = D / K, NTN = (D + 31) / 32;
  using Op = typename std::conditional<G::W16, u32x4, float>::type;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 5, l32 = lane & 31;
  const int rt = 4 / ep, rtile = wave % rt, part = wave / rt;  // row tile, E part
  const int h = blockIdx.x / tiles_per_head, bt = blockIdx.x % tiles_per_head;
  const int b0 = bt * (32 * rt) + rtile * 32;
  const long long B = a.B, E = a.E;
  const long long xb = h * a.sx[0], db = h * a.sdo[0], w1b = h * a.sw1[0], w2b = h * a.sw2[0];

  // X^T / dO^T operands: lane = row b0 + l32, k-slots d; loaded once for the whole E loop where
  // they fit next to the dX accumulators (16-bit io up to D = 128, fp32 up to D = 64), else per chunk
  constexpr bool HOIST = G::W16 ? D <= 128 : D <= 64;
  const int bx = b0 + l32;
  const long long rx = xb + (long long)bx * a.sx[1], rd = db + (long long)bx * a.sdo[1];
  auto rows = [&](int ks, Op& xo, Op& dq) {
    if constexpr (G::W16) {
      xo = row_op16(a.x, rx, opaque(a.sx[2]), ks, g, bx < B, a.vec_x);
      dq = row_op16(a.dout, rd, opaque(a.sdo[2]), ks, g, bx < B, a.vec_do);
    } else {
      xo = bx < B ? ld32(a.x, rx + (long long)(2 * ks + g) * opaque(a.sx[2])) : 0.f;
      dq = bx < B ? ld32(a.dout, rd + (long long)(2 * ks + g) * opaque(a.sdo[2])) : 0.f;
    }
  };
  Op xr[HOIST ? KS : 1], dr[HOIST ? KS : 1];
  if constexpr (HOIST) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) rows(ks, xr[ks], dr[ks]);
  }
  f32x16 acc[NTN];
#pragma unroll
  for (int nt = 0; nt < NTN; ++nt) acc[nt] = zero16();

  for (long long c0 = 32LL * part; c0 < E; c0 += 32LL * ep) {
    const long long sw11 = opaque(a.sw1[1]), sw12 = opaque(a.sw1[2]);
    const long long sw21 = opaque(a.sw2[1]), sw22 = opaque(a.sw2[2]);
    const long long e = c0 + l32;
    f32x16 z = zero16(), dh = zero16();
    // Z^T, dH^T (M = e, N = b): A = W1c^T / W2c (lane = column e), B = X^T / dO^T rows
    struct G1 {
      Op a1, a2, x, d;
    };
    pipelined<KS, G1>(
        [&](int ks) {
          G1 o;
          if constexpr (G::W16) {
            o.a1 = op16(e < E, [&](int j) { return ld16(a.w1, w1b + (long long)(ks * 16 + 8 * g + j) * sw11 + e * sw12); });
            o.a2 = row_op16(a.w2, w2b + e * sw21, sw22, ks, g, e < E, a.vec_w2);
          } else {
            o.a1 = e < E ? ld32(a.w1, w1b + (long long)(2 * ks + g) * sw11 + e * sw12) : 0.f;
            o.a2 = e < E ? ld32(a.w2, w2b + e * sw21 + (long long)(2 * ks + g) * sw22) : 0.f;
          }
          if constexpr (!HOIST) rows(ks, o.x, o.d);
          return o;
        },
        [&](int ks, const G1& o) {
          const Op xo = HOIST ? xr[HOIST ? ks : 0] : o.x, dq = HOIST ? dr[HOIST ? ks : 0] : o.d;
          if constexpr (G::W16) {
            z = mma16(G::BF, o.a1, xo, z);
            dh = mma16(G::BF, o.a2, dq, dh);
          } else {
            z = mma32(o.a1, xo, z);
            dh = mma32(o.a2, dq, dh);
          }
        });
    float dz[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float hh, dd;
      act_fb_rt(a.act, z[i], dh[i], hh, dd);
      dz[i] = io_round<IO>(dd);
    }
    // dX += dZ W1c^T: B = W1c^T, lane = column d, k-slots e (in dZ's order)
    if constexpr (G::W16) {
      u32x4 zA[2];
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int w = 0; w < 4; ++w) zA[s][w] = pack2<G::BF>(dz[8 * s + 2 * w], dz[8 * s + 2 * w + 1]);
      pipelined<2 * NTN, u32x4>(
          [&](int q) {
            const int nt = q >> 1, s = q & 1, d = nt * 32 + l32;
            // k-slots j: columns c0 + 16 s + 4 g + (j & 3) + 8 (j / 4), two runs of four
            const long long ec = c0 + 16 * s + 4 * g;
            u32x4 Bv = {0u, 0u, 0u, 0u};
            if (a.vec_w1 && ec + 11 < E) {  // wave-uniform flag; both runs inside E
              if (d < D) {
                const u16* rowp = (const u16*)a.w1 + w1b + (long long)d * sw11 + ec;
                Bv = cat(*(const u32x2*)rowp, *(const u32x2*)(rowp + 8));
              }
            } else {
              Bv = op16(d < D, [&](int j) {
                const long long ee = ec + 8 * (j / 4) + (j & 3);
                return ee < E ? ld16(a.w1, w1b + (long long)d * sw11 + ee * sw12) : 0u;
              });
            }
            return Bv;
          },
          [&](int q, const u32x4& Bv) { acc[q >> 1] = mma16(G::BF, zA[q & 1], Bv, acc[q >> 1]); });
    } else {
      pipelined<16 * NTN, float>(
          [&](int q) {
            const int nt = q >> 4, i = q & 15, d = nt * 32 + l32;
            const long long ee = c0 + 8 * (i / 4) + 4 * g + (i & 3);
            return (d < D && ee < E) ? ld32(a.w1, w1b + (long long)d * sw11 + ee * sw12) : 0.f;
          },
          [&](int q, const float& Bv) { acc[q >> 4] = mma32(dz[q & 15], Bv, acc[q >> 4]); });
    }
  }
  gen_sum_parts<NTN>(acc, ep, part, rtile, rt, lane);
  if (part > 0) return;
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
  using Op = typename std::conditional<G::W16, u32x4, float>::type;
  // the wave's W1c / W2c^T operands stay in registers for the whole row loop where they fit
  // next to the dW accumulators (16-bit io up to D = 128, fp32 up to D = 64)
  constexpr bool HOIST = G::W16 ? D <= 128 : D <= 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 5, l32 = lane & 31;
  // workgroup = (head, 128-column E-tile, B range s of rows_per_split rows)
  constexpr int DH = gen_dw_dsplit(D), NTW = NTN / DH, CG = 4 / DH;
  const int cg = wave % CG, half = wave / CG;  // column group, D half (nt range half * NTW ..)
  const int hs = blockIdx.x / a.nS, sp = blockIdx.x % a.nS;
  const int h = hs / tiles_per_head, et = hs % tiles_per_head;
  const long long e0 = (long long)et * gen_dw_cols(D) + cg * 32;
  const long long B = a.B, E = a.E;
  const long long b_lo = (long long)sp * a.rows_per_split;
  const long long b_hi = a.nS > 1 ? (b_lo + a.rows_per_split < B ? b_lo + a.rows_per_split : B) : B;
  const long long xb = h * a.sx[0], db = h * a.sdo[0], w1b = h * a.sw1[0], w2b = h * a.sw2[0];
  const long long e = e0 + l32;  // this lane's column in Z / dH

  auto wop = [&](int ks, long long sw11, long long sw12, long long sw21, long long sw22, Op& B1, Op& B2) {
    if constexpr (G::W16) {
      B1 = op16(e < E, [&](int j) { return ld16(a.w1, w1b + (long long)(ks * 16 + 8 * g + j) * sw11 + e * sw12); });
      B2 = row_op16(a.w2, w2b + e * sw21, sw22, ks, g, e < E, a.vec_w2);
    } else {
      const long long d = 2 * ks + g;
      B1 = e < E ? ld32(a.w1, w1b + d * sw11 + e * sw12) : 0.f;
      B2 = e < E ? ld32(a.w2, w2b + e * sw21 + d * sw22) : 0.f;
    }
  };
  Op w1r[HOIST ? KS : 1], w2r[HOIST ? KS : 1];
  if constexpr (HOIST) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) wop(ks, a.sw1[1], a.sw1[2], a.sw2[1], a.sw2[2], w1r[ks], w2r[ks]);
  }

  f32x16 a1[NTW], a2[NTW];  // dW1^T and dW2 (M = e, N = d) of the wave's D tiles
#pragma unroll
  for (int t = 0; t < NTW; ++t) {
    a1[t] = zero16();
    a2[t] = zero16();
  }
  for (long long r0 = b_lo; r0 < b_hi; r0 += 32) {
    const long long sx1 = opaque(a.sx[1]), sx2 = opaque(a.sx[2]), sdo1 = opaque(a.sdo[1]), sdo2 = opaque(a.sdo[2]);
    // Z, dH (M = rows, N = e): A = X / dO rows (lane = row r0 + l32), B = W1c / W2c^T (lane = e)
    const long long rA = r0 + l32;
    f32x16 z = zero16(), dh = zero16();
    struct G1 {
      Op ax, ad, b1, b2;
    };
    pipelined<KS, G1>(
        [&](int ks) {
          G1 o;
          if constexpr (G::W16) {
            o.ax = row_op16(a.x, xb + rA * sx1, sx2, ks, g, rA < B, a.vec_x);
            o.ad = row_op16(a.dout, db + rA * sdo1, sdo2, ks, g, rA < B, a.vec_do);
          } else {
            const long long d = 2 * ks + g;
            o.ax = rA < B ? ld32(a.x, xb + rA * sx1 + d * sx2) : 0.f;
            o.ad = rA < B ? ld32(a.dout, db + rA * sdo1 + d * sdo2) : 0.f;
          }
          if constexpr (!HOIST) wop(ks, opaque(a.sw1[1]), opaque(a.sw1[2]), opaque(a.sw2[1]), opaque(a.sw2[2]), o.b1, o.b2);
          return o;
        },
        [&](int ks, const G1& o) {
          const Op B1 = HOIST ? w1r[HOIST ? ks : 0] : o.b1, B2 = HOIST ? w2r[HOIST ? ks : 0] : o.b2;
          if constexpr (G::W16) {
            z = mma16(G::BF, o.ax, B1, z);
            dh = mma16(G::BF, o.ad, B2, dh);
          } else {
            z = mma32(o.ax, B1, z);
            dh = mma32(o.ad, B2, dh);
          }
        });
    // h, dZ: lane = column e, value i = row r0 + 8 (i / 4) + 4 g + i % 4 (rows past B: X, dO
    // are zero there, so dZ = 0 and h multiplies a zero dO row)
    // (16-bit io rounds h and dZ when packing them into the operands below)
    float hv[16], dz[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) act_fb_rt(a.act, z[i], dh[i], hv[i], dz[i]);
    // dW2 += h^T dO, dW1^T += dZ^T X: A from h / dZ (lane = e), B = dO / X (lane = column d,
    // k-slots rows in h's order)
    if constexpr (G::W16) {
      u32x4 Ah[2], Az[2], AhL[2], AzL[2];  // io-rounded terms, and the lo terms v - round(v) (hilo)
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float h0 = hv[8 * s + 2 * w], h1 = hv[8 * s + 2 * w + 1];
          const float z0 = dz[8 * s + 2 * w], z1 = dz[8 * s + 2 * w + 1];
          Ah[s][w] = pack2<G::BF>(h0, h1);
          Az[s][w] = pack2<G::BF>(z0, z1);
          AhL[s][w] = pack2<G::BF>(h0 - lo_f32<G::BF>(Ah[s][w]), h1 - hi_f32<G::BF>(Ah[s][w]));
          AzL[s][w] = pack2<G::BF>(z0 - lo_f32<G::BF>(Az[s][w]), z1 - hi_f32<G::BF>(Az[s][w]));
        }
      pipelined<2 * NTW, Pair<u32x4>>(
          [&](int q) {
            const int t = q >> 1, s = q & 1, d = (half * NTW + t) * 32 + l32;
            auto row = [&](int j) { return r0 + 16 * s + 8 * (j / 4) + 4 * g + (j & 3); };
            Pair<u32x4> o;
            o.a = op16(d < D, [&](int j) {
              const long long r = row(j);
              return r < B ? ld16(a.dout, db + r * sdo1 + (long long)d * sdo2) : 0u;
            });
            o.b = op16(d < D, [&](int j) {
              const long long r = row(j);
              return r < B ? ld16(a.x, xb + r * sx1 + (long long)d * sx2) : 0u;
            });
            return o;
          },
          [&](int q, const Pair<u32x4>& o) {
            const int t = q >> 1, s = q & 1;
            a2[t] = mma16(G::BF, Ah[s], o.a, a2[t]);
            a1[t] = mma16(G::BF, Az[s], o.b, a1[t]);
            if (a.hilo) {
              a2[t] = mma16(G::BF, AhL[s], o.a, a2[t]);
              a1[t] = mma16(G::BF, AzL[s], o.b, a1[t]);
            }
          });
    } else {
      pipelined<16 * NTW, Pair<float>>(
          [&](int q) {
            const int t = q >> 4, i = q & 15, d = (half * NTW + t) * 32 + l32;
            const long long r = r0 + 8 * (i / 4) + 4 * g + (i & 3);
            const bool ok = d < D && r < B;
            Pair<float> o;
            o.a = ok ? ld32(a.dout, db + r * sdo1 + (long long)d * sdo2) : 0.f;
            o.b = ok ? ld32(a.x, xb + r * sx1 + (long long)d * sx2) : 0.f;
            return o;
          },
          [&](int q, const Pair<float>& o) {
            const int t = q >> 4, i = q & 15;
            a2[t] = mma32(hv[i], o.a, a2[t]);
            a1[t] = mma32(dz[i], o.b, a1[t]);
          });
    }
  }
  // dW2[h][e][d], dW1[h][d][e]: lane = column d, value i = row e0 + 8 (i / 4) + 4 g + i % 4;
  // with a B split, fp32 partials in the same layouts in slice sp of the workspace
  const long long per = a.H * E * D;
  float* p2 = a.nS > 1 ? (float*)a.ws + (long long)sp * per : nullptr;
  float* p1 = a.nS > 1 ? (float*)a.ws + (long long)(a.nS + sp) * per : nullptr;
#pragma unroll
  for (int t = 0; t < NTW; ++t) {
    const int d = (half * NTW + t) * 32 + l32;
    if (d < D) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const long long ee = e0 + 8 * (i / 4) + 4 * g + (i & 3);
        if (ee < E) {
          const long long i2 = ((long long)h * E + ee) * D + d, i1 = ((long long)h * D + d) * E + ee;
          if (a.nS > 1) {
            p2[i2] = a2[t][i];
            p1[i1] = a1[t][i];
          } else {
            st_out<IO>(a.dw2, i2, a2[t][i], a.out_f32);
            st_out<IO>(a.dw1, i1, a1[t][i], a.out_f32);
          }
        }
      }
    }
  }
}

// Sum of the B split's fp32 partials (dW2 slices, then dW1 slices, each in its output's dense
// layout) in split order, so the result is deterministic; rounded to the io dtype at the store
// (or kept fp32 for fp32 io / FMLP_OUT_F32).
template <int IO>
__global__ void __launch_bounds__(256) gen_dw_reduce_kernel(const float* __restrict__ ws, void* __restrict__ dW1,
                                                            void* __restrict__ dW2, long long per, int nS, int outf32) {
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long q = (long long)blockIdx.x * blockDim.x + threadIdx.x; q < 2 * per; q += stride) {
    const bool second = q >= per;  // false: dW2, true: dW1
    const long long i = second ? q - per : q;
    const float* src = ws + (second ? (long long)nS * per : 0) + i;
    float acc = src[0];
    for (int s = 1; s < nS; ++s) acc += src[(long long)s * per];
    st_out<IO>(second ? dW1 : dW2, i, acc, outf32);
  }
}

// ------------------------------------------------------------------------------------
// launchers
// ------------------------------------------------------------------------------------
namespace {

// E parts per workgroup of the forward / dX kernels: the fewest (1, 2, 4) whose grid of
// H ceil(B / (32 (4 / ep))) workgroups covers the CUs, within the LDS the partial sums need
int gen_eparts(long long H, long long B, int D, int num_cus) {
  int ep = 1;
  while (ep < 4 && H * ((B + 32LL * (4 / ep) - 1) / (32LL * (4 / ep))) < num_cus) ep *= 2;
  const int ntn = (D + 31) / 32;
  while (ep > 1 && (size_t)(ep - 1) * (4 / ep) * ntn * 4096 > 96u * 1024u) ep /= 2;
  return ep;
}

template <typename K>
hipError_t gen_launch_rows(K kern, const GenArgs& a, int D, hipStream_t st, std::atomic<unsigned long long>& lds_set) {
  const int ep = gen_eparts(a.H, a.B, D, a.num_cus);
  const long long tph = (a.B + 32LL * (4 / ep) - 1) / (32LL * (4 / ep));
  const long long grid = tph * a.H;
  if (grid <= 0) return hipSuccess;
  if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
  const size_t lds = (size_t)(ep - 1) * (4 / ep) * ((D + 31) / 32) * 4096;
  if (lds > 0) {
    const hipError_t e = set_lds_once((const void*)kern, 96 * 1024, lds_set);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(GEN_NT), lds, st, a, (int)tph, ep);
  return hipGetLastError();
}

template <int IO, int D>
hipError_t gen_launch_fwd_t(const GenArgs& a, hipStream_t st) {
  static std::atomic<unsigned long long> lds_set{0};
  return gen_launch_rows(gen_fwd_kernel<IO, D>, a, D, st, lds_set);
}

template <int IO, int D>
hipError_t gen_launch_bwd_t(const GenArgs& a, hipStream_t st) {
  const long long tph = (a.B + GEN_ROWS - 1) / GEN_ROWS;
  const long long ctph = (a.E + gen_dw_cols(D) - 1) / gen_dw_cols(D);
  const long long ns = a.nS > 1 ? a.nS : 1;
  if (tph * a.H > 0x7fffffffLL || ctph * a.H * ns > 0x7fffffffLL) return hipErrorInvalidValue;
  if (ns > 1 && (a.ws == nullptr || a.rows_per_split <= 0 || a.rows_per_split % 32 != 0)) return hipErrorInvalidValue;
  if (a.H > 0 && ctph > 0 && a.want_dw) {
    hipLaunchKernelGGL((gen_dw_kernel<IO, D>), dim3((unsigned)(ctph * a.H * ns)), dim3(GEN_NT), 0, st, a, (int)ctph);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (ns > 1) {
      const long long per = a.H * a.E * a.D;
      long long blocks = (2 * per + 255) / 256;
      if (blocks > 8192) blocks = 8192;
      hipLaunchKernelGGL((gen_dw_reduce_kernel<IO>), dim3((unsigned)blocks), dim3(256), 0, st, (const float*)a.ws,
                         a.dw1, a.dw2, per, (int)ns, a.out_f32);
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
  }
  if (a.H > 0 && tph > 0 && a.want_dx) {
    static std::atomic<unsigned long long> lds_set{0};
    return gen_launch_rows(gen_dx_kernel<IO, D>, a, D, st, lds_set);
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

// About two dW workgroups per CU, at least 128 rows per B range; the largest such split whose
// fp32 partials (2 nS H E D floats) fit max_ws, else none.
GenPlan gen_plan(int64_t H, int64_t B, int64_t D, int64_t E, int num_cus, size_t max_ws) {
  GenPlan p{1, 0, 0};
  const int cols = gen_dw_cols((int)D);
  const long long base = H * ((E + cols - 1) / cols);
  if (base <= 0 || B <= 0) return p;
  const long long N = num_cus > 0 ? num_cus : 1;
  long long ns = (2 * N + base - 1) / base;
  const long long max_ns = B / 128 > 1 ? B / 128 : 1;
  if (ns > max_ns) ns = max_ns;
  for (; ns > 1; --ns) {
    long long rps = (B + ns - 1) / ns;
    rps = (rps + 31) / 32 * 32;
    const long long eff = (B + rps - 1) / rps;
    if (eff <= 1) continue;
    const size_t bytes = (size_t)2 * (size_t)eff * (size_t)H * (size_t)E * (size_t)D * sizeof(float);
    if (bytes <= max_ws) {
      p.nS = (int)eff;
      p.rows_per_split = (int)rps;
      p.ws_bytes = bytes;
      return p;
    }
  }
  return p;
}

}  // namespace fmlp
