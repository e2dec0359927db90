// FlashMLP backward kernels for gfx950 (MI355X).
//
// The reference's two program roles (flashmlp.py:360-373). bwd_kernel holds both in one
// launch, split by workgroup id (the role with the longer programs first).
//   * dW programs (dw2_body): per head, 128-column E-tile and B-range;
//     recompute Z = X W1c and dH = dO W2c^T per 32-row subtile, then dW2 += h^T dO and
//     dW1^T += dZ^T X (flashmlp.py:247-329). h and dZ are cast to the io dtype before those
//     contractions (flashmlp.py:297-320) and come straight from the MFMA C layout
//     (lane = E column).
//   * dX programs (dx2_body): per head and 256-row B-tile;
//     recompute Z^T and dH^T = W2c dO^T per 32-column E-chunk, dZ = dH * act'(Z) cast to the
//     io dtype, and dX += dZ W1c^T (flashmlp.py:165-244).
//   * dw_reduce_kernel sums the dW programs' fp32 partials when B is split.
// Leaky ReLU uses the autograd slope at Z == 0 (0.01); the reference Triton kernel uses 1.
#include "fmlp_device.h"
#include "fmlp_launch.h"
#include <algorithm>
#include <cmath>
#include <mutex>
#include <type_traits>

namespace fmlp {

constexpr int DW_ET = 128;           // E columns per dW program (32 per wave column group)
constexpr int DW_BT = 32;            // rows per streamed subtile

// dW epilogue. C layout of the accumulators: lane = column d
// (32 nt + l32), rows e = e0 + 8 (i / 4) + 4 g + (i % 4). nS == 1 writes dW1, dW2 in the io
// dtype (fp32 when outf32); otherwise fp32 partials in the outputs' layouts, ws2[s][h][e][d]
// and ws1[s][h][d][e], which dw_reduce_kernel sums elementwise.
template <bool BF16, int D>
__device__ __forceinline__ void dw_store(const f32x16 (&a1)[D / 32], const f32x16 (&a2)[D / 32], void* __restrict__ dW1,
                                         void* __restrict__ dW2, float* __restrict__ ws, int H, int E, int h, int s,
                                         int nS, int e0, int g, int l32, int outf32) {
  constexpr int NTN = D / 32;
  if (nS == 1 && outf32) {
    float* dW2h = (float*)dW2 + (size_t)h * E * D;
    float* dW1h = (float*)dW1 + (size_t)h * D * E;
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      const int eb = e0 + 8 * i4 + 4 * g;
      if (eb < E) {
#pragma unroll
        for (int nt = 0; nt < NTN; ++nt) {
          const int d = nt * 32 + l32;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            dW2h[(size_t)(eb + j) * D + d] = a2[nt][4 * i4 + j];
            dW1h[(size_t)d * E + eb + j] = a1[nt][4 * i4 + j];
          }
        }
      }
    }
  } else if (nS == 1) {
    u16* dW2h = (u16*)dW2 + (size_t)h * E * D;
    u16* dW1h = (u16*)dW1 + (size_t)h * D * E;
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      const int eb = e0 + 8 * i4 + 4 * g;  // 4 consecutive columns eb .. eb+3 (E % 8 == 0)
      if (eb < E) {
#pragma unroll
        for (int nt = 0; nt < NTN; ++nt) {
          const int d = nt * 32 + l32;
#pragma unroll
          for (int j = 0; j < 4; ++j) dW2h[(size_t)(eb + j) * D + d] = from_f32<BF16>(a2[nt][4 * i4 + j]);
          u32x2 v = {pack2<BF16>(a1[nt][4 * i4 + 0], a1[nt][4 * i4 + 1]), pack2<BF16>(a1[nt][4 * i4 + 2], a1[nt][4 * i4 + 3])};
          *(u32x2*)(dW1h + (size_t)d * E + eb) = v;
        }
      }
    }
  } else {
    // fp32 partials in the outputs' own layouts (dW2 [h][e][d], dW1 [h][d][e]), so the
    // reduction is an elementwise sum over the nS slices
    const size_t per = (size_t)H * E * D;
    float* p2 = ws + ((size_t)s * H + h) * E * D;
    float* p1 = ws + (size_t)nS * per + ((size_t)s * H + h) * D * E;
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      const int eb = e0 + 8 * i4 + 4 * g;  // 4 consecutive columns eb .. eb+3 (E % 8 == 0)
      if (eb < E) {
#pragma unroll
        for (int nt = 0; nt < NTN; ++nt) {
          const int d = nt * 32 + l32;
#pragma unroll
          for (int j = 0; j < 4; ++j) p2[(size_t)(eb + j) * D + d] = a2[nt][4 * i4 + j];
          const float4 v = {a1[nt][4 * i4], a1[nt][4 * i4 + 1], a1[nt][4 * i4 + 2], a1[nt][4 * i4 + 3]};
          *(float4*)(p1 + (size_t)d * E + eb) = v;
        }
      }
    }
  }
}

// ------------------------------------------------------------------------------------
// dX programs, two-waves-per-SIMD form (dx2_kernel): 8 waves x 32 rows = 256 rows of one
// head. Per 32-column E-chunk c each wave runs two phases:
//   MFMA phase: Z^T(c) = W1c^T X^T and dH^T(c) = W2c dO^T (16 MFMAs) interleaved with
//               dX += dZ(c-1) W1c(c-1)^T (8 MFMAs), operand reads three steps ahead;
//   VALU phase: dZ(c) = dH * act'(Z) for the wave's 32 x 32 tile, cast to the io dtype.
// Waves 0-3 run MFMA-then-VALU, waves 4-7 VALU(c-1)-then-MFMA, so the two waves sharing a
// SIMD keep the matrix cores and the VALU busy at the same time (the per-chunk barrier
// would otherwise align them). Nothing is double-buffered in registers, which keeps a wave
// within 256 VGPRs. W1c / W2c chunks go straight from global memory into an 8-slot LDS ring
// (buffer loads with the LDS destination, DX_PF = 4 chunks ahead of the chunk read).
//
// E-order inside a chunk: Z^T row m holds chunk column e = sig(m) (bits 2 and 3 of m
// swapped). Then the 8 k-slots a lane holds of the dZ operand (C layout rows
// 16 s + 8 (j / 4) + 4 g + j % 4) are 8 consecutive columns 16 s + 8 g + j, and the W1c
// operand of dX is one 16-byte row read. The transposed W1c^T read and the W2c row read
// pick their columns / rows in the same order.
//
// LDS slot (128 D bytes): W1c [D rows d][32 columns e] 64-byte rows, 16-byte chunk q of row
// r at chunk q ^ ((r >> 2) & 3); then W2c [32 rows e][D] as D/32 blocks of [32][32]
// (w2s_off). Both are written as lane-linear 16-byte pieces; each lane loads the global
// piece that belongs at its LDS position.
// ------------------------------------------------------------------------------------
__device__ __forceinline__ constexpr unsigned sig(unsigned m) {
  return (m & ~12u) | ((m & 4u) << 1) | ((m & 8u) >> 1);
}

constexpr int DX2_NW = 8;
constexpr int DX2_NT = DX2_NW * 64;
constexpr int DX2_ROWS = DX2_NW * 32;
constexpr int DX_NSLOT = 8;  // chunk ring slots (128 D bytes each)
constexpr int DX_PF = 4;     // chunks requested ahead of the one read
static_assert(DX_PF <= DX_NSLOT - 2, "a slot is reloaded only after the barrier that retires its last reader");
// At D = 256 (dX only; the dW role's tiles do not fit the LDS there) a program is 4 waves of 32
// rows at one wave per SIMD, and a chunk is 32 KB: a 4-slot ring two chunks ahead.
__host__ __device__ constexpr int dx_nslot(int D) { return D <= 128 ? DX_NSLOT : 4; }
__host__ __device__ constexpr int dx_pf(int D) { return D <= 128 ? DX_PF : 2; }

// DES = 2 (E split, D = 64 only: grids of 256-row dX programs that leave CUs idle): a program
// owns 128 rows; waves 0-3 walk the first half of the E-chunks and waves 4-7 the second, each
// half through an LDS ring of its own, and the second half's partial dX tile is added to the
// first's through LDS at the end.
template <int D, int DES>
__host__ __device__ constexpr int dx2_rows() { return DX2_ROWS / DES; }

// A program owns tile t's rows and the E-chunks [cb, ce); with pws set (a ragged tile split
// over E) it stores its fp32 partial dX tile there ([rows][D]) instead of writing dX.
template <bool BF16, int D, int ACT, int DES = 1, int NW = DX2_NW>
__device__ __forceinline__ void dx2_body(const u16* __restrict__ X, const u16* __restrict__ W1,
                                         const u16* __restrict__ W2, const u16* __restrict__ dO,
                                         void* __restrict__ dX, int B, int E, int tiles_per_head, int outf32,
                                         int t, int cb, int ce, float* __restrict__ pws) {
  static_assert(DES == 1 || (DES == 2 && D == 64), "E split");
  static_assert(NW == DX2_NW || (NW == 4 && D == 256 && DES == 1), "waves per program");
  constexpr int KS = D / 16, NTN = D / 32;
  constexpr unsigned SLOT = 128u * D;
  constexpr unsigned W2OFF = 64u * D;
  constexpr int NTP = NW * 64 / DES;     // threads of one E part
  constexpr int ROWS = NW * 32 / DES;    // rows per program
  constexpr int NDMA = 8 * D / NTP;      // 16-byte pieces per lane per chunk
  constexpr int N1 = 2 * KS, N2 = 2 * NTN;
  constexpr int PD = 3;
  constexpr int NSL = dx_nslot(D), PF = dx_pf(D);
  static_assert(PF <= NSL - 2 && NDMA * NTP == 8 * D, "ring and pieces");

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform for the compiler
  const int G = lane >> 4, i16 = lane & 15, g = lane >> 5, l32 = lane & 31;
  const int part = DES == 1 ? 0 : wave >> 2;       // E part
  const int wp = DES == 1 ? wave : (wave & 3);     // wave within the part

  const int h = t / tiles_per_head, bt = t - h * tiles_per_head;
  const int NC = ce - cb;
  const int NCP = (NC + DES - 1) / DES;             // chunks per part: global chunk c0 + ci
  const int c0 = cb + part * NCP;
  const int e_end = min(E, ce * 32);                // columns of W1 (rows of W2) read
  const int RB = part * NSL * (int)SLOT;            // this part's ring
  // VALU-first half of the workgroup (the second part when split); with one wave per SIMD
  // (NW = 4) every wave runs the MFMA-first order
  const bool late = NW == 8 && wave >= 4;

  const u16* Xh = X + (size_t)h * B * D;
  const u16* dOh = dO + (size_t)h * B * D;
  const u16* W1h = W1 + (size_t)h * D * E;
  const u16* W2h = W2 + (size_t)h * E * D;
  const int b_wave = bt * ROWS + wp * 32;

  // ---- staging pieces: piece p (16 bytes at slot offset 16 p) of a chunk ----
  unsigned dmaOff[NDMA];
  int dmaCol[NDMA];  // W1c pieces: first chunk column (masked against E); W2c pieces: -1
#pragma unroll
  for (int k = 0; k < NDMA; ++k) {
    const unsigned p = k * NTP + wp * 64 + lane;
    if (p < 4u * D) {  // W1c row r, logical chunk q
      const unsigned r = p >> 2, q = (p & 3u) ^ ((r >> 2) & 3u);
      dmaOff[k] = r * (unsigned)E * 2u + q * 16u;
      dmaCol[k] = (int)(q * 8u);
    } else {           // W2c block bk, row rr, logical piece q
      const unsigned pp = p - 4u * D, bk = pp >> 7, rr = (pp >> 2) & 31u;
      const unsigned q = bk * 4u + ((pp & 3u) ^ ((rr >> 2) & 3u));
      dmaOff[k] = rr * (D * 2u) + q * 16u;
      dmaCol[k] = -1;
    }
  }
  // chunk staging: buffer-to-LDS loads PF chunks ahead into an NSL-slot ring; part chunk
  // ci is global chunk c0 + ci, and chunks past the part's share (or past the range) load as zeros
  auto dma_chunk = [&](int ci) {
    const int c = c0 + ci;
    const bool mine = ci < NCP;
    const int lim = mine ? e_end - c * 32 : 0;
    const int rem = mine ? D * E * 2 - 64 * c : 0;
    const i32x4 r1 = make_rsrc_words(W1h + (size_t)c * 32, rem > 0 ? rem : 0);
    const i32x4 r2 = make_rsrc_words(W2h + (size_t)c * 32 * D, clamp0(lim, 32) * D * 2);
    const int slot = RB + (ci & (NSL - 1)) * (int)SLOT + wp * 1024;
#pragma unroll
    for (int k = 0; k < NDMA; ++k) {
      // W1c or W2c piece (wave-uniform): word-wise selects keep the loop body one basic block
      const bool w1 = (unsigned)(k * NTP + wp * 64) < 4u * D;
      i32x4 rr;
#pragma unroll
      for (int i = 0; i < 4; ++i) rr[i] = __builtin_amdgcn_readfirstlane(w1 ? r1[i] : r2[i]);
      buf_load16_lds(rr, dmaCol[k] < lim ? dmaOff[k] : BUF_OOB, slot + k * NTP * 16);
    }
  };

  // ---- X and dO rows in registers: B operand (lane = row b, 8 consecutive d) ----
  u32x4 xr[KS], dr[KS];
  {
    const int b = b_wave + l32;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4 v = {0u, 0u, 0u, 0u}, w = {0u, 0u, 0u, 0u};
      if (b < B) {
        v = *(const u32x4*)(Xh + (size_t)b * D + ks * 16 + g * 8);
        w = *(const u32x4*)(dOh + (size_t)b * D + ks * 16 + g * 8);
      }
      xr[ks] = v;
      dr[ks] = w;
    }
  }

  // ---- per-lane LDS offsets (slot relative) ----
  // Z^T A operand (W1c^T), two transposed reads r = 0, 1: lane 4j + q of a 16-lane group
  // reads row 16 ks + 8 g + 4 r + j, columns from 16 (G % 2) + 8 (q % 2) + 4 (q / 2);
  // the row's swizzle is (2 g + r) & 3 for every ks.
  unsigned offA[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const unsigned j = i16 >> 2, q = i16 & 3;
    const unsigned chunk = 2u * (G & 1) + (q & 1u);
    offA[r] = (8u * g + 4u * r + j) * 64u + ((chunk ^ ((2u * g + r) & 3u)) << 4) + 8u * (q >> 1);
  }
  // dH^T A operand: W2c row sig(l32), piece 2 ks + g -> offW2[ks % 2] + (ks / 2) * 2048
  unsigned offW2[2];
#pragma unroll
  for (int kp = 0; kp < 2; ++kp) offW2[kp] = W2OFF + w2s_off(sig(l32), 2 * kp + g);
  // dX B operand: W1c row 32 nt + l32, piece 2 s + g -> offB[s] + nt * 2048
  unsigned offB[2];
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2) offB[s2] = l32 * 64u + (((2u * s2 + g) ^ ((l32 >> 2) & 3u)) << 4);

  f32x16 acc[NTN];
#pragma unroll
  for (int nt = 0; nt < NTN; ++nt) acc[nt] = zero16();
  f32x16 z = zero16(), dh = zero16();
  u32x4 dz[2];

  // MFMA phase over chunk c (G1: Z^T(c), dH^T(c)) and, when G2, chunk c - 1 (dX += dZ W1c^T)
  auto mfma_phase = [&](auto G2, int c) {
    constexpr bool DO_G2 = decltype(G2)::value;
    constexpr int M2 = DO_G2 ? N2 : 0, NOPS = N1 + M2;
    const int base1 = RB + (c & (NSL - 1)) * (int)SLOT, base2 = RB + ((c - 1) & (NSL - 1)) * (int)SLOT;
    auto fetch = [&](int j) -> u32x4 {
      const int q = sched_index(j, N1, M2);
      if (sched_is_g2(j, N1, M2)) {
        const int s2 = q / NTN, nt = q % NTN;
        return lds_read16(base2 + (int)offB[s2] + nt * 2048);
      }
      const int ks = q >> 1;
      if ((q & 1) == 0)
        return cat(lds_read_tr(base1 + (int)offA[0] + ks * 1024), lds_read_tr(base1 + (int)offA[1] + ks * 1024));
      return lds_read16(base1 + (int)offW2[ks & 1] + (ks >> 1) * 2048);
    };
    u32x4 ring[PD + 1];
#pragma unroll
    for (int j = 0; j < PD; ++j) ring[j] = fetch(j);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < NOPS; ++j) {
      const u32x4 cur = ring[j % (PD + 1)];
      if (j + PD < NOPS) ring[(j + PD) % (PD + 1)] = fetch(j + PD);
      const int q = sched_index(j, N1, M2);
      if (sched_is_g2(j, N1, M2)) {
        const int s2 = q / NTN, nt = q % NTN;
        acc[nt] = mfma<BF16>(dz[s2], cur, acc[nt]);
      } else {
        const int ks = q >> 1;  // ks == 0 starts the chain from a literal zero accumulator
        if ((q & 1) == 0) z = mfma<BF16>(cur, xr[ks], ks == 0 ? zero16() : z);
        else dh = mfma<BF16>(cur, dr[ks], ks == 0 ? zero16() : dh);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto g2_only = [&](int c) {  // dX += dZ(c) W1c(c)^T
    const int base2 = RB + (c & (NSL - 1)) * (int)SLOT;
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int nt = 0; nt < NTN; ++nt) acc[nt] = mfma<BF16>(dz[s2], lds_read16(base2 + (int)offB[s2] + nt * 2048), acc[nt]);
  };
  auto valu_phase = [&]() {
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int w = 0; w < 4; ++w)
        dz[s2][w] = pack2<BF16>(act_b<ACT>(z[8 * s2 + 2 * w], dh[8 * s2 + 2 * w]),
                                act_b<ACT>(z[8 * s2 + 2 * w + 1], dh[8 * s2 + 2 * w + 1]));
    __builtin_amdgcn_sched_barrier(0);
  };
  // iteration c requests chunk c + PF; the end-of-chunk barrier publishes chunk c + 1 (each
  // wave waits for its own pieces first) and retires every read of chunk c - 1, whose slot
  // holds chunk c - 1 + NSL later
  auto chunk_begin = [&](int c) { dma_chunk(c + PF); };
  auto chunk_end = [&]() {
    wait_vmcnt<NDMA * (PF - 1)>();
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    asm volatile("" ::: "memory");       // keep LDS accesses on their side of the barrier
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

#pragma unroll
  for (int c = 0; c < PF; ++c) dma_chunk(c);
  chunk_end();
  const std::true_type T{};
  const std::false_type F{};
  // (chunk indices below are part-relative; both parts run NCP iterations, so the workgroup
  // barriers line up)
  if (!late) {
    chunk_begin(0);
    mfma_phase(F, 0);
    valu_phase();
    chunk_end();
    for (int c = 1; c < NCP; ++c) {
      mfma_phase(T, c);
      chunk_begin(c);  // staged between the phases: fewer LDS writes next to the operand reads
      valu_phase();
      chunk_end();
    }
  } else {
    chunk_begin(0);
    mfma_phase(F, 0);
    chunk_end();
    for (int c = 1; c < NCP; ++c) {
      chunk_begin(c);
      valu_phase();
      mfma_phase(T, c);
      chunk_end();
    }
    valu_phase();
  }
  g2_only(NCP - 1);
  wait_vmcnt<0>();  // chunk loads past the last are still landing (as zeros)
  if constexpr (DES == 2) {  // part 1 hands its partial dX tile to part 0 through LDS (the rings)
    asm volatile("" ::: "memory");
    __syncthreads();
    const int ob = wp * (NTN * 4096);  // per wave NTN x 4 x [64 lanes][16 bytes]
    if (part == 1) {
#pragma unroll
      for (int nt = 0; nt < NTN; ++nt)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4)
          lds_write16(ob + ((nt * 4 + i4) * 64 + lane) * 16,
                      u32x4{__float_as_uint(acc[nt][4 * i4]), __float_as_uint(acc[nt][4 * i4 + 1]),
                            __float_as_uint(acc[nt][4 * i4 + 2]), __float_as_uint(acc[nt][4 * i4 + 3])});
    }
    __syncthreads();
    if (part == 1) return;
#pragma unroll
    for (int nt = 0; nt < NTN; ++nt)
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const u32x4 v = lds_read16(ob + ((nt * 4 + i4) * 64 + lane) * 16);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[nt][4 * i4 + j] += __uint_as_float(v[j]);
      }
  }
  if (pws != nullptr)
    store_rows<BF16, D>(acc, pws, 0, B - bt * ROWS, wp * 32, g, l32, 1);
  else
    store_rows<BF16, D>(acc, dX, (size_t)h * B * D, B, b_wave, g, l32, outf32);
}

// ------------------------------------------------------------------------------------
// dW programs, two-waves-per-SIMD form (dw2_kernel): 8 waves per (head, 128-column E-tile,
// B-range). Waves w and w + 4 share a SIMD and the E-columns 32 (w % 4) .. + 31 and take
// alternate 32-row subtiles (set 0 = waves 0-3 the even ones, set 1 the odd ones); their
// dW partial sums are added through LDS at the end. The E-tile's W1c^T and W2c are kept
// in LDS (no room in registers next to both dW accumulators), so every Z / dH MFMA reads
// both operands from LDS:
//   W1T [128 e][D] and W2T [128 e][D] : D/32 blocks of [128 rows][64 bytes], 16-byte chunk
//       q of row r at chunk q ^ ((r >> 2) & 3) (wt_off), read row-wise (lane = column e);
//   ring of 3 slots, each a subtile pair [X set0][dO set0][X set1][dO set1] of [32][D]
//       in the w2s_off layout, written by lane-linear buffer-to-LDS loads one pair ahead.
// Per pair each wave computes Z, dH of its subtile (16 MFMAs), then h, dZ interleaved with
// dW2 += h^T dO and dW1^T += dZ^T X over the same subtile (16 MFMAs); set 0 does this for
// the current pair, set 1 finishes the previous pair first, so the two waves of a SIMD
// are half a pair apart.
// ------------------------------------------------------------------------------------
constexpr int DW2_NW = 8;
constexpr int DW2_NT = DW2_NW * 64;

// weight tile of ET rows: D/32 blocks of [ET rows][64 bytes]
template <int ET>
__device__ __forceinline__ unsigned wt_off(unsigned r, unsigned q) {
  return (q >> 2) * (ET * 64u) + r * 64u + (((q & 3u) ^ ((r >> 2) & 3u)) << 4);
}

// HILO: the dW products take h and dZ as two io-dtype terms, hi = round(v) and
// lo = round(v - hi), instead of round(v) alone (twice the dW MFMAs, same operand reads);
// an accuracy mode with no counterpart in the reference, whose kernel rounds h and dZ to
// the io dtype (flashmlp.py:297-320).
// DZ: the programs also store dZ (the io-dtype value the dX product takes) to dzt in the image
// dxg_kernel streams into LDS: [h][b / 256][e / 32][(b % 256) / 32][e % 32][32 positions], row
// b at position sig(b % 32) (bits 2 and 3 swapped), so each 32-column chunk of a 256-row tile
// is 16 contiguous KB.
// ET: E-columns per program, 128 (four column groups of waves, two row sets: the form
// described above) or 64 (D = 64, recompute form only: two column groups, four row sets, wave
// w taking every fourth subtile of its set; twice the programs, each half the work, for grids
// that leave CUs idle). Waves w and w + 4 share a SIMD; their sets differ by RS / 2, so one
// runs the schedule half a group behind the other either way.
template <bool BF16, int D, int ACT, bool HILO, bool DZ = false, int ET = DW_ET>
__device__ __forceinline__ void dw2_body(const u16* __restrict__ X, const u16* __restrict__ W1,
                                         const u16* __restrict__ W2, const u16* __restrict__ dO,
                                         void* __restrict__ dW1, void* __restrict__ dW2, float* __restrict__ ws,
                                         int H, int B, int E, int nE, int nS, int rows_per_split, int outf32,
                                         int t, u16* __restrict__ dzt = nullptr, int Bp = 0) {
  static_assert(ET == DW_ET || (ET == 64 && D == 64 && !DZ), "E-tile width");
  constexpr int KS = D / 16, NTN = D / 32;
  constexpr int CG = ET / 32;            // column groups of waves
  constexpr int RS = DW2_NW / CG;        // row sets (a set takes every RS-th subtile)
  constexpr int SUB = 64 * D;            // bytes of a [32][D] subtile
  constexpr int PAIR = 2 * RS * SUB;     // a group of subtiles: X set0, dO set0, X set1, dO set1, ...
  constexpr int WT = 2 * ET * D;         // bytes of an [ET][D] weight tile
  constexpr int WTB = ET * 64;           // bytes of one 32-column block of it
  // ring first (its runtime slot base plus constant offsets stays within the 16-bit DS
  // immediate range), weight tiles above it (addressed from a lane register that holds
  // the tile base)
  constexpr int RING_OFF = 0, W1T_OFF = 3 * PAIR, W2T_OFF = W1T_OFF + WT;
  constexpr int NPL = PAIR / 16 / DW2_NT;  // 16-byte pieces per lane per group
  static_assert(PAIR % (16 * DW2_NT) == 0 && (ET * D / 8) % DW2_NT == 0, "piece counts");
  constexpr int N1 = 2 * KS, N2 = 4 * NTN;
  constexpr int PD = 2;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = lane >> 4, i16 = lane & 15, g = lane >> 5, l32 = lane & 31;
  const int cg = wave % CG, set = wave / CG;
  const int et = t % nE;
  const int hs = t / nE;
  const int s = hs % nS, h = hs / nS;
  const int e_prog = et * ET;
  const int e0 = e_prog + 32 * cg;
  const int b_lo = s * rows_per_split;
  const int b_hi = min(B, b_lo + rows_per_split);
  const int nsub = (b_hi - b_lo + DW_BT - 1) / DW_BT;
  const int npair = (nsub + RS - 1) / RS;

  const u16* Xh = X + (size_t)h * B * D;
  const u16* dOh = dO + (size_t)h * B * D;
  const u16* W1h = W1 + (size_t)h * D * E;
  const u16* W2h = W2 + (size_t)h * E * D;

  // ---- weight tiles (once): W2T rows natural, W1T transposed with 2-byte writes ----
#pragma unroll
  for (int k = 0; k < ET * D / 8 / DW2_NT; ++k) {
    const int p = tid + k * DW2_NT;
    {  // W2 row e_prog + r, piece q
      const int r = p / (D / 8), q = p % (D / 8);
      u32x4 v = {0u, 0u, 0u, 0u};
      if (e_prog + r < E) v = *(const u32x4*)(W2h + (size_t)(e_prog + r) * D + q * 8);
      lds_write16(W2T_OFF + (int)wt_off<ET>(r, q), v);
    }
    {  // W1 row d, columns e_prog + 8u .. + 7  ->  W1T rows 8u + j, column d
      const int d = p / (ET / 8), u = p % (ET / 8);
      u32x4 v = {0u, 0u, 0u, 0u};
      if (e_prog + 8 * u < E) v = *(const u32x4*)(W1h + (size_t)d * E + e_prog + 8 * u);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const u16 x = (u16)(v[j >> 1] >> (16 * (j & 1)));
        *(FMLP_LDS u16*)((FMLP_LDS char*)fmlp_lds + W1T_OFF + wt_off<ET>(8 * u + j, d >> 3) + (d & 7) * 2) = x;
      }
    }
  }

  // ---- subtile pairs: lane-linear buffer-to-LDS pieces ----
  unsigned pieceOff[NPL];
#pragma unroll
  for (int k = 0; k < NPL; ++k) {
    const unsigned p = k * DW2_NT + wave * 64 + lane, pr = p % (SUB / 16), o = 16u * pr;
    const unsigned r = (o % 2048u) / 64u, q = 4u * (o / 2048u) + (((o / 16u) & 3u) ^ ((r >> 2) & 3u));
    pieceOff[k] = r * (D * 2u) + q * 16u;
  }
  auto issue_pair = [&](int i, int slot) {
#pragma unroll
    for (int k = 0; k < NPL; ++k) {
      const int region = (k * DW2_NT + wave * 64) / (SUB / 16);  // wave-uniform: 2 s X of set s, 2 s + 1 dO
      const int r0 = b_lo + (RS * i + (region >> 1)) * DW_BT;
      const int bytes = clamp0(b_hi - r0, DW_BT) * D * 2;
      const i32x4 rs = make_rsrc_words(((region & 1) ? dOh : Xh) + (size_t)r0 * D, bytes);
      buf_load16_lds(rs, pieceOff[k], RING_OFF + slot * PAIR + 16 * (k * DW2_NT + wave * 64));
    }
  };

  // ---- per-lane LDS offsets ----
  const int own = set * 2 * SUB;  // this wave's subtile inside a pair: X at own, dO at own + SUB
  //   A operand of Z / dH: subtile row l32, piece 2 ks + g -> offRow[ks % 2] + (ks / 2) * 2048
  int offRow[2];
#pragma unroll
  for (int kp = 0; kp < 2; ++kp) offRow[kp] = own + (int)w2s_off(l32, 2 * kp + g);
  //   B operand of Z / dH: weight-tile row 32 cg + l32, piece 2 ks + g -> offWt[ks % 2] + (ks / 2) * 8192
  int offWt[2];
#pragma unroll
  for (int kp = 0; kp < 2; ++kp) offWt[kp] = W1T_OFF + (int)wt_off<ET>(32 * cg + l32, 2 * kp + g);
  //   B operand of dW2 / dW1^T (transposed subtile reads) -> offTr[r] + nt * 2048 + s * 1024
  int offTr[2];
#pragma unroll
  for (int r = 0; r < 2; ++r)
    offTr[r] = own + (int)(w2s_off(8 * r + 4 * g + (i16 >> 2), 2 * (G & 1) + ((i16 & 3) >> 1)) + 8u * (i16 & 1));

  f32x16 a2[NTN], a1[NTN];
#pragma unroll
  for (int nt = 0; nt < NTN; ++nt) {
    a2[nt] = zero16();
    a1[nt] = zero16();
  }
  f32x16 z = zero16(), dh = zero16();
  u32x4 hT[2], dzT[2];
  u32x4 hL[2], dzL[2];  // lo terms (HILO only)

  struct Opnd {
    u32x4 a, b;
  };
  // Z and dH of the wave's subtile of the pair in `slot`: 16 MFMAs, both operands from LDS,
  // read PD steps ahead
  auto g1_phase = [&](int slot) {
    const int base = RING_OFF + slot * PAIR;
    auto fetch = [&](int q) -> Opnd {
      const int ks = q >> 1, which = q & 1;  // which 0 -> Z (X, W1T), 1 -> dH (dO, W2T)
      Opnd o;
      o.a = lds_read16(base + (which ? SUB : 0) + offRow[ks & 1] + (ks >> 1) * 2048);
      o.b = lds_read16((which ? WT : 0) + offWt[ks & 1] + (ks >> 1) * WTB);
      return o;
    };
    Opnd ring[PD + 1];
#pragma unroll
    for (int j = 0; j < PD; ++j) ring[j] = fetch(j);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < N1; ++q) {
      const Opnd cur_op = ring[q % (PD + 1)];
      if (q + PD < N1) ring[(q + PD) % (PD + 1)] = fetch(q + PD);
      const int ks = q >> 1;  // ks == 0 starts the chain from a literal zero accumulator
      if ((q & 1) == 0) z = mfma<BF16>(cur_op.a, cur_op.b, ks == 0 ? zero16() : z);
      else dh = mfma<BF16>(cur_op.a, cur_op.b, ks == 0 ? zero16() : dh);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // h, dZ of the subtile whose Z, dH are in registers, and dW2 += h^T dO, dW1^T += dZ^T X
  // over it (its pair is in `slot`). Elements 0-7 (the K-step-0 operands) are activated
  // first; the 8 K-step-0 MFMAs then run with elements 8-15 spread between them, and the
  // 8 K-step-1 MFMAs follow.
  // per-head dZ resource (DZ): Bp / 256 tiles of [nE * 128 rows e][256 positions]
  const int Ep = nE * ET;
  const u16* dzh = DZ ? dzt + (size_t)h * Ep * Bp : nullptr;
  // lane part of the dZ store offsets inside a subtile's 2 KB block [32 columns][32 positions]
  unsigned dzLane[2];
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2) dzLane[s2] = ((unsigned)l32 * 32u + (unsigned)(16 * s2 + 8 * g)) * 2u;
  auto ag2_phase = [&](int slot, int rbase) {
    const int base2 = RING_OFF + slot * PAIR;
    auto fetch = [&](int q) -> u32x4 {  // (s, nt, which): which 0 -> dW2 (B = dO^T), 1 -> dW1^T (B = X^T)
      const int s2 = q / (2 * NTN), nt = (q % (2 * NTN)) >> 1, which = q & 1;
      const int bb = base2 + (which == 0 ? SUB : 0) + nt * 2048 + s2 * 1024;
      return cat(lds_read_tr(bb + offTr[0]), lds_read_tr(bb + offTr[1]));
    };
    auto act_elem = [&](int e, float (&hv)[16], float (&dv)[16]) {
      act_fb<ACT>(z[e], dh[e], hv[e], dv[e]);
      if (e & 1) {
        const unsigned ph = pack2<BF16>(hv[e - 1], hv[e]), pd = pack2<BF16>(dv[e - 1], dv[e]);
        hT[e >> 3][(e >> 1) & 3] = ph;
        dzT[e >> 3][(e >> 1) & 3] = pd;
        if constexpr (HILO) {  // v - round(v) is exact in fp32; its rounding is the lo term
          hL[e >> 3][(e >> 1) & 3] = pack2<BF16>(hv[e - 1] - lo_f32<BF16>(ph), hv[e] - hi_f32<BF16>(ph));
          dzL[e >> 3][(e >> 1) & 3] = pack2<BF16>(dv[e - 1] - lo_f32<BF16>(pd), dv[e] - hi_f32<BF16>(pd));
        }
      }
    };
    float hv[16], dv[16];
    u32x4 ring[PD + 1];
#pragma unroll
    for (int j = 0; j < PD; ++j) ring[j] = fetch(j);
#pragma unroll
    for (int e = 0; e < 8; ++e) act_elem(e, hv, dv);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < N2; ++q) {
      const u32x4 cur_op = ring[q % (PD + 1)];
      if (q + PD < N2) ring[(q + PD) % (PD + 1)] = fetch(q + PD);
      const int s2 = q / (2 * NTN), nt = (q % (2 * NTN)) >> 1;
      if ((q & 1) == 0) {
        a2[nt] = mfma<BF16>(hT[s2], cur_op, a2[nt]);
        if constexpr (HILO) a2[nt] = mfma<BF16>(hL[s2], cur_op, a2[nt]);
      } else {
        a1[nt] = mfma<BF16>(dzT[s2], cur_op, a1[nt]);
        if constexpr (HILO) a1[nt] = mfma<BF16>(dzL[s2], cur_op, a1[nt]);
      }
#pragma unroll
      for (int e = 8 + sched_elem_begin(q, N2 / 2, 8); e < 8 + sched_elem_begin(q + 1, N2 / 2, 8); ++e)
        if (e < 16) act_elem(e, hv, dv);
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (DZ) {
      // dzT[s] holds rows 16 s + 4 g + 0..3 and 16 s + 8 + 4 g + 0..3 of column e0 + l32: positions
      // 16 s + 8 g .. + 7 under sig, one 16-byte store each; subtiles past the program's rows
      // (the odd last one of a B range) store nothing (an empty resource). The block base and
      // that test are wave-uniform, so they live in the resource (scalar registers) and each
      // lane's offset is a constant.
      const bool live = rbase < b_hi;
      const unsigned blk = ((unsigned)(rbase >> 8) * (unsigned)(Ep >> 5) + (unsigned)(e0 >> 5)) * 8u +
                           (unsigned)((rbase & 255) >> 5);
      const Rsrc rb = make_rsrc(dzh + (size_t)blk * 1024u, live ? 2048 : 0);
#pragma unroll
      // non-temporal: dZ is read once, by dxg_kernel, so its lines should not stay in the
      // device's caches (measured at cfg4: backward -20 us, step +1.4 %)
      for (int s2 = 0; s2 < 2; ++s2)
        __builtin_amdgcn_raw_buffer_store_b128(dzT[s2], rb, (int)dzLane[s2], 0, CPOL_NT);
    }
  };
  // end of a pair: this wave's loads of the next pair have landed; the barrier publishes
  // them and retires every read of the slot the pair after reuses
  // (DZ: the two dZ stores of the ag2 phase issued after those loads may stay in flight)
  auto pair_end = [&](auto AFTER_AG2) {
    wait_vmcnt<(DZ && decltype(AFTER_AG2)::value) ? 2 : 0>();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  const std::true_type AG{};
  const std::false_type NOAG{};
  if (npair > 0) {
    issue_pair(0, 0);
    pair_end(NOAG);  // also publishes the weight tiles
    int cur = 0, prev = 2, next = 1;  // ring slots of pairs i, i - 1, i + 1
    auto rotate = [&]() {
      const int tmp = prev;
      prev = cur;
      cur = next;
      next = tmp;
    };
    issue_pair(1, next);
    g1_phase(cur);
    // first row of the subtile set `set` takes in group i
    auto row0 = [&](int i) { return b_lo + (RS * i + set) * DW_BT; };
    if (set < RS / 2) {
      ag2_phase(cur, row0(0));
      pair_end(AG);
      for (int i = 1; i < npair; ++i) {
        rotate();
        issue_pair(i + 1, next);
        g1_phase(cur);
        ag2_phase(cur, row0(i));
        pair_end(AG);
      }
    } else {
      pair_end(NOAG);
      for (int i = 1; i < npair; ++i) {
        rotate();
        issue_pair(i + 1, next);
        ag2_phase(prev, row0(i - 1));
        g1_phase(cur);
        pair_end(AG);
      }
      ag2_phase(cur, row0(npair - 1));
    }
  } else {
    wait_vmcnt<0>();
  }

  // ---- add the sets' partial sums through LDS (sets 1 .. RS-1 write, set 0 adds them in order) ----
  asm volatile("" ::: "memory");
  __syncthreads();
  {
    constexpr int ACCB = 2 * NTN * 16 * 256;  // 2 NTN accumulators x 16 registers x 64 lanes x 4 bytes
    const int xb = ((set > 0 ? set - 1 : 0) * CG + cg) * ACCB;
    if (set > 0) {
#pragma unroll
      for (int nt = 0; nt < NTN; ++nt)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
          u32x4 v2 = {__float_as_uint(a2[nt][4 * i4]), __float_as_uint(a2[nt][4 * i4 + 1]), __float_as_uint(a2[nt][4 * i4 + 2]), __float_as_uint(a2[nt][4 * i4 + 3])};
          u32x4 v1 = {__float_as_uint(a1[nt][4 * i4]), __float_as_uint(a1[nt][4 * i4 + 1]), __float_as_uint(a1[nt][4 * i4 + 2]), __float_as_uint(a1[nt][4 * i4 + 3])};
          lds_write16(xb + ((nt * 4 + i4) * 64 + lane) * 16, v2);
          lds_write16(xb + (((NTN + nt) * 4 + i4) * 64 + lane) * 16, v1);
        }
    }
    __syncthreads();
    if (set == 0) {
#pragma unroll
      for (int so = 1; so < RS; ++so) {
        const int sb = ((so - 1) * CG + cg) * ACCB;
#pragma unroll
        for (int nt = 0; nt < NTN; ++nt)
#pragma unroll
          for (int i4 = 0; i4 < 4; ++i4) {
            const u32x4 v2 = lds_read16(sb + ((nt * 4 + i4) * 64 + lane) * 16);
            const u32x4 v1 = lds_read16(sb + (((NTN + nt) * 4 + i4) * 64 + lane) * 16);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              a2[nt][4 * i4 + j] += __uint_as_float(v2[j]);
              a1[nt][4 * i4 + j] += __uint_as_float(v1[j]);
            }
          }
      }
      dw_store<BF16, D>(a1, a2, dW1, dW2, ws, H, E, h, s, nS, e0, g, l32, outf32);
    }
  }
}

// dX programs as their own launch (FMLP_BWD_UNIFIED=0, FMLP_BWD_NO_DW): 8 waves, two per SIMD.
template <bool BF16, int D, int ACT, int DES>
__global__ void __launch_bounds__(DX2_NT) __attribute__((amdgpu_waves_per_eu(2, 2)))
dx2_kernel(const u16* __restrict__ X, const u16* __restrict__ W1, const u16* __restrict__ W2,
           const u16* __restrict__ dO, void* __restrict__ dX, int B, int E, int tiles_per_head, int outf32) {
  dx2_body<BF16, D, ACT, DES>(X, W1, W2, dO, dX, B, E, tiles_per_head, outf32, xcd_remap(blockIdx.x, gridDim.x), 0,
                              (E + 31) >> 5, nullptr);
}

// dX programs at D = 256 (the tuned backward's dX only; its dW runs on the generic kernels):
// 4 waves of 32 rows, one per SIMD (the X and dO rows and the dX accumulators take ~320
// registers of the 512).
template <bool BF16, int ACT>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
dx256_kernel(const u16* __restrict__ X, const u16* __restrict__ W1, const u16* __restrict__ W2,
             const u16* __restrict__ dO, void* __restrict__ dX, int B, int E, int tiles_per_head, int outf32) {
  dx2_body<BF16, 256, ACT, 1, 4>(X, W1, W2, dO, dX, B, E, tiles_per_head, outf32, xcd_remap(blockIdx.x, gridDim.x),
                                 0, (E + 31) >> 5, nullptr);
}

// ------------------------------------------------------------------------------------
// dW programs at D = 256 (dw256_kernel): 4 waves, one per SIMD. A program owns 128 E-columns
// of one head (wave w the 32 columns e0 = e_prog + 32 w) and a B-range of rows_per_split
// rows, as a dw2_body program does. The 512 registers of a lone wave hold its two
// accumulators (dW2 and dW1^T, [32 e][256 d] each: 256) and, loaded once, its weight operands:
// the B operands of Z = X W1c and dH = dO W2c^T for its columns (lane = column e0 + l32,
// k-slots d = 16 ks + 8 g + j; 128). Only X and dO pass through LDS: per 32-row subtile
// 32 KB in a 4-slot ring filled by buffer-to-LDS loads DW4_PF subtiles ahead and read by all
// four waves. Per subtile a wave issues 64 MFMAs in one operand stream:
//   Z = X W1c (16, a chain), dH = dO W2c^T (16) with h = act(Z) and act'(Z) of elements
//   0-11 between them, dW2 += h^T dO (16) with elements 12-15 and then dZ = dH act'(Z)
//   between them, dW1^T += dZ^T X (16)
// (the dW products twice with HILO). Subtile layout and operand reads are dw2_body's
// (w2s_off blocks; row reads for the A operands of Z and dH, ds_read_b64_tr_b16 for the B
// operands of the dW products). W1c reaches its register layout through LDS once: a
// row-major [256 d][128 e] staging tile in the ring's last two slots, read transposed before
// the ring first uses them; W2c rows are loaded straight into registers.
// ------------------------------------------------------------------------------------
constexpr int DW4_NSLOT = 4;                   // subtile ring slots
constexpr int DW4_PF = 3;                      // subtiles requested ahead of the one read
constexpr int DW4_SUB = 32 * 256 * 2;          // bytes of one [32][256] tile (X or dO)
constexpr int DW4_SLOT = 2 * DW4_SUB;          // a slot: the X tile, then the dO tile
constexpr int DW4_NPL = DW4_SLOT / 16 / 256;   // 16-byte pieces per lane per subtile
constexpr int DW4_PD = 3;                      // operand reads ahead of their MFMA
static_assert(DW4_PF <= DW4_NSLOT - 1, "a slot is reloaded only after the barrier that retires its last reader");
static_assert(DW4_PF >= 2 && 2 * DW4_SLOT == 256 * DW_ET * 2, "the W1c staging tile fills the ring's last two slots");
static_assert(16 % (DW4_PD + 1) == 0, "each 16-step group starts at ring slot 0");

// h = act(z) and the factor f with dZ = dH f (act_fb's arithmetic, split in two so that h can be
// computed before dH is)
template <int ACT>
__device__ __forceinline__ void act_hf(float z, float& h, float& f) {
  if constexpr (ACT == ACT_SILU) {
    const float s = sigm(z);
    h = z * s;
    f = __builtin_fmaf(h, 1.0f - s, s);
  } else if constexpr (ACT == ACT_LEAKY) {
    const bool p = z > 0.f;
    h = p ? z : 0.01f * z;
    f = p ? 1.0f : 0.01f;
  } else if constexpr (ACT == ACT_SIGMOID) {
    const float s = sigm(z);
    h = s;
    f = s - s * s;
  } else {
    h = z;
    f = 1.0f;
  }
}

template <bool BF16, int ACT, bool HILO>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
dw256_kernel(const u16* __restrict__ X, const u16* __restrict__ W1, const u16* __restrict__ W2,
             const u16* __restrict__ dO, void* __restrict__ dW1, void* __restrict__ dW2, float* __restrict__ ws,
             int H, int B, int E, int nE, int nS, int rows_per_split, int outf32) {
  constexpr int D = 256, KS = D / 16, NTN = D / 32;
  constexpr int STG = 2 * DW4_SLOT;  // W1c staging tile: [256 d][128 e], 256-byte rows
  constexpr int PD = DW4_PD;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = lane >> 4, i16 = lane & 15, g = lane >> 5, l32 = lane & 31;
  const int t = xcd_remap(blockIdx.x, gridDim.x);
  const int et = t % nE, hs = t / nE;
  const int s = hs % nS, h = hs / nS;
  const int e_prog = et * DW_ET, e0 = e_prog + 32 * wave;
  const int b_lo = s * rows_per_split;
  const int b_hi = min(B, b_lo + rows_per_split);
  const int nsub = b_hi > b_lo ? (b_hi - b_lo + DW_BT - 1) / DW_BT : 0;

  const u16* Xh = X + (size_t)h * B * D;
  const u16* dOh = dO + (size_t)h * B * D;
  const u16* W1h = W1 + (size_t)h * D * E;
  const u16* W2h = W2 + (size_t)h * E * D;

  // ---- subtile loads: lane-linear 16-byte pieces (pieces k4 of the X tile, then of dO) ----
  unsigned pieceOff[4];
#pragma unroll
  for (int k4 = 0; k4 < 4; ++k4) {
    const unsigned pr = k4 * 256 + wave * 64 + lane, o = 16u * pr, r = (o % 2048u) / 64u;
    const unsigned q = 4u * (o / 2048u) + (((o / 16u) & 3u) ^ ((r >> 2) & 3u));
    pieceOff[k4] = r * (D * 2u) + q * 16u;
  }
  // subtile i (rows b_lo + 32 i ..) into slot i % 4; rows at or past b_hi read as zeros (an
  // empty resource past the range), which add nothing to either product
  auto issue = [&](int i) {
    const int slot = i & (DW4_NSLOT - 1);
    const int r0 = b_lo + i * DW_BT;
    const int bytes = clamp0(b_hi - r0, DW_BT) * D * 2;
    const i32x4 rx = make_rsrc_words(Xh + (size_t)r0 * D, bytes);
    const i32x4 rd = make_rsrc_words(dOh + (size_t)r0 * D, bytes);
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4)
      buf_load16_lds(rx, pieceOff[k4], slot * DW4_SLOT + 16 * (k4 * 256 + wave * 64));
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4)
      buf_load16_lds(rd, pieceOff[k4], slot * DW4_SLOT + DW4_SUB + 16 * (k4 * 256 + wave * 64));
  };
  issue(0);
  issue(1);

  // ---- weight operands (once) ----
  // W1 rows d, columns e_prog .. + 127 -> staging tile (zeros past E; E % 8 == 0)
#pragma unroll 4
  for (int k = 0; k < 256 * 16 / 256; ++k) {
    const int p = tid + 256 * k, d = p >> 4, u = p & 15;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (e_prog + 8 * u < E) v = *(const u32x4*)(W1h + (size_t)d * E + e_prog + 8 * u);
    lds_write16(STG + d * 256 + u * 16, v);
  }
  // W2 row e0 + l32, d = 16 ks + 8 g .. + 7: the B operand of dH as it lies in memory
  u32x4 w2op[KS];
  const bool col_ok = e0 + l32 < E;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (col_ok) v = *(const u32x4*)(W2h + (size_t)(e0 + l32) * D + 16 * ks + 8 * g);
    w2op[ks] = v;
  }
  __syncthreads();
  // W1c B operand: ds_read_b64_tr_b16 over 4 rows d x 16 columns e of the staging tile gives
  // lane i16 of each 16-lane group column 32 wave + 16 (G & 1) + i16, rows d .. d + 3
  u32x4 w1op[KS];
  {
    const int c2 = (32 * wave + 16 * (G & 1) + 4 * (i16 & 3)) * 2;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int d0 = 16 * ks + 8 * g + (i16 >> 2);
      w1op[ks] = cat(lds_read_tr(STG + d0 * 256 + c2), lds_read_tr(STG + (d0 + 4) * 256 + c2));
    }
  }
  // the staging reads have returned (lgkmcnt 0) and subtiles 0 and 1 have landed before the
  // barrier that hands the staging slots to the ring
  __builtin_amdgcn_s_waitcnt(0xC07F);
  wait_vmcnt<0>();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
#pragma unroll
  for (int i = 2; i < DW4_PF; ++i) issue(i);

  // ---- per-lane LDS offsets inside a slot ----
  //   A operand of Z / dH: row l32, piece 2 ks + g -> offRow[ks % 2] + (ks / 2) * 2048
  int offRow[2];
#pragma unroll
  for (int kp = 0; kp < 2; ++kp) offRow[kp] = (int)w2s_off(l32, 2 * kp + g);
  //   B operand of dW2 / dW1^T (transposed reads) -> offTr[r] + nt * 2048 + s2 * 1024
  int offTr[2];
#pragma unroll
  for (int r = 0; r < 2; ++r)
    offTr[r] = (int)(w2s_off(8 * r + 4 * g + (i16 >> 2), 2 * (G & 1) + ((i16 & 3) >> 1)) + 8u * (i16 & 1));

  f32x16 a2[NTN], a1[NTN];
#pragma unroll
  for (int nt = 0; nt < NTN; ++nt) {
    a2[nt] = zero16();
    a1[nt] = zero16();
  }
  f32x16 z = zero16(), dh = zero16();
  u32x4 hT[2], dzT[2], hL[2], dzL[2];  // lo terms: HILO only

  for (int i = 0; i < nsub; ++i) {
    issue(i + DW4_PF);  // into the slot of subtile i - 1, retired by the last barrier
    const int base = (i & (DW4_NSLOT - 1)) * DW4_SLOT;
    // operand q of the subtile's 64 MFMAs: X rows (Z), dO rows (dH), dO^T (dW2), X^T (dW1^T)
    auto fetch = [&](int q) -> u32x4 {
      if (q < 32) {
        const int ks = q & 15;
        return lds_read16(base + (q < 16 ? 0 : DW4_SUB) + offRow[ks & 1] + (ks >> 1) * 2048);
      }
      const int qq = q & 15, s2 = qq >> 3, nt = qq & 7;
      const int bb = base + (q < 48 ? DW4_SUB : 0) + nt * 2048 + s2 * 1024;
      return cat(lds_read_tr(bb + offTr[0]), lds_read_tr(bb + offTr[1]));
    };
    float hv[16], fv[16], dv[16];
    auto vh = [&](int e) {  // h and act' of element e
      act_hf<ACT>(z[e], hv[e], fv[e]);
      if (e & 1) {
        const unsigned ph = pack2<BF16>(hv[e - 1], hv[e]);
        hT[e >> 3][(e >> 1) & 3] = ph;
        if constexpr (HILO)  // v - round(v) is exact in fp32; its rounding is the lo term
          hL[e >> 3][(e >> 1) & 3] = pack2<BF16>(hv[e - 1] - lo_f32<BF16>(ph), hv[e] - hi_f32<BF16>(ph));
      }
    };
    auto vd = [&](int e) {  // dZ of element e
      dv[e] = dh[e] * fv[e];
      if (e & 1) {
        const unsigned pd = pack2<BF16>(dv[e - 1], dv[e]);
        dzT[e >> 3][(e >> 1) & 3] = pd;
        if constexpr (HILO)
          dzL[e >> 3][(e >> 1) & 3] = pack2<BF16>(dv[e - 1] - lo_f32<BF16>(pd), dv[e] - hi_f32<BF16>(pd));
      }
    };
    u32x4 ring[PD + 1];
#pragma unroll
    for (int j = 0; j < PD; ++j) ring[j] = fetch(j);
    __builtin_amdgcn_sched_barrier(0);
    // four groups of 16 steps (each loop unrolls fully, so every index below is a constant);
    // step q takes ring slot q % 4 (16 is a multiple of PD + 1) and reads operand q + PD
    auto next = [&](int q) {
      if (q + PD < 64) ring[(q + PD) % (PD + 1)] = fetch(q + PD);
    };
#pragma unroll
    for (int k = 0; k < 16; ++k) {  // Z = X W1c
      const u32x4 op = ring[k % (PD + 1)];
      next(k);
      z = mfma<BF16>(op, w1op[k], k == 0 ? zero16() : z);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) {  // dH = dO W2c^T; h and act' of elements 0-11
      const u32x4 op = ring[k % (PD + 1)];
      next(16 + k);
      dh = mfma<BF16>(op, w2op[k], k == 0 ? zero16() : dh);
#pragma unroll
      for (int e = sched_elem_begin(k, 16, 12); e < sched_elem_begin(k + 1, 16, 12); ++e) vh(e);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) {  // dW2 += h^T dO; elements 12-15, then dZ
      const u32x4 op = ring[k % (PD + 1)];
      next(32 + k);
      const int s2 = k >> 3, nt = k & 7;
      a2[nt] = mfma<BF16>(hT[s2], op, a2[nt]);
      if constexpr (HILO) a2[nt] = mfma<BF16>(hL[s2], op, a2[nt]);
      if (k < 8) {
#pragma unroll
        for (int e = 12 + sched_elem_begin(k, 8, 4); e < 12 + sched_elem_begin(k + 1, 8, 4); ++e) vh(e);
      } else {
#pragma unroll
        for (int e = sched_elem_begin(k - 8, 8, 16); e < sched_elem_begin(k - 7, 8, 16); ++e) vd(e);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) {  // dW1^T += dZ^T X
      const u32x4 op = ring[k % (PD + 1)];
      next(48 + k);
      const int s2 = k >> 3, nt = k & 7;
      a1[nt] = mfma<BF16>(dzT[s2], op, a1[nt]);
      if constexpr (HILO) a1[nt] = mfma<BF16>(dzL[s2], op, a1[nt]);
      __builtin_amdgcn_sched_barrier(0);
    }
    // subtile i + 1 has landed (this wave's part; the barrier publishes the others' and retires
    // every read of slot i, which subtile i + 4 reuses)
    wait_vmcnt<(DW4_PF - 1) * DW4_NPL>();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  }
  wait_vmcnt<0>();  // the empty requests past the range
  dw_store<BF16, D>(a1, a2, dW1, dW2, ws, H, E, h, s, nS, e0, g, l32, outf32);
}

template <bool BF16, int D, int ACT, bool HILO, bool DZ, int ET = DW_ET>
__global__ void __launch_bounds__(DW2_NT) __attribute__((amdgpu_waves_per_eu(2, 2)))
dw2_kernel(const u16* __restrict__ X, const u16* __restrict__ W1, const u16* __restrict__ W2,
           const u16* __restrict__ dO, void* __restrict__ dW1, void* __restrict__ dW2, float* __restrict__ ws,
           int H, int B, int E, int nE, int nS, int rows_per_split, int outf32, u16* __restrict__ dzt, int Bp) {
  dw2_body<BF16, D, ACT, HILO, DZ, ET>(X, W1, W2, dO, dW1, dW2, ws, H, B, E, nE, nS, rows_per_split, outf32,
                                   xcd_remap(blockIdx.x, gridDim.x), dzt, Bp);
}

// Unified backward launch (flashmlp.py:341-421's program-id split): the role whose programs
// run longer comes first in workgroup order (dW programs [0, n_dw) then dX programs, or dX
// first when dx_first), so the shorter programs fill the CUs that finish early. Both roles
// use 8 waves (two per SIMD); the dynamic LDS is the dW role's (the larger). Each role's
// tiles are remapped onto XCDs within its own range (exact when its count is a multiple of 8).
static_assert(DW2_NT == DX2_NT, "both roles run with the same workgroup size");
template <bool BF16, int D, int ACT, bool HILO, int DES, int ET = DW_ET>
__global__ void __launch_bounds__(DW2_NT) __attribute__((amdgpu_waves_per_eu(2, 2)))
bwd_kernel(const u16* __restrict__ X, const u16* __restrict__ W1, const u16* __restrict__ W2,
           const u16* __restrict__ dO, void* __restrict__ dX, void* __restrict__ dW1, void* __restrict__ dW2,
           float* __restrict__ ws, int H, int B, int E, int nE, int nS, int rows_per_split, int n_dw,
           int dx_tiles_per_head, int dx_first, int outf32, int n_dxs, int dxs_xs, int dxs_nct,
           float* __restrict__ dxs_ws) {
  // programs: n_dw dW programs and n_dx whole-tile dX programs (in the plan's order), then
  // n_dxs = H dxs_xs programs for the heads' ragged last dX tiles split over E (when the plan
  // splits them, the whole-tile dX programs are the other tiles: T - 1 per head)
  const int b = blockIdx.x, n_rest = (int)gridDim.x - n_dxs, n_dx = n_rest - n_dw;
  const int T = dx_tiles_per_head, nch = (E + 31) >> 5;
  if (b >= n_rest) {
    const int u = b - n_rest, hh = u / dxs_xs, cb = (u - hh * dxs_xs) * dxs_nct;
    dx2_body<BF16, D, ACT, DES>(X, W1, W2, dO, dX, B, E, T, outf32, hh * T + T - 1, cb, min(nch, cb + dxs_nct),
                                dxs_ws + (size_t)u * dx2_rows<D, DES>() * D);
    return;
  }
  const int bw = dx_first ? b - n_dx : b;  // index among the dW programs (< 0 or >= n_dw: a dX program)
  if (bw >= 0 && bw < n_dw) {
    dw2_body<BF16, D, ACT, HILO, false, ET>(X, W1, W2, dO, dW1, dW2, ws, H, B, E, nE, nS, rows_per_split, outf32,
                                            xcd_remap(bw, n_dw));
  } else {
    const int bx = dx_first ? b : b - n_dw;
    const int m = xcd_remap(bx, n_dx);
    const int t = n_dxs > 0 ? (m / (T - 1)) * T + m % (T - 1) : m;
    dx2_body<BF16, D, ACT, DES>(X, W1, W2, dO, dX, B, E, T, outf32, t, 0, nch, nullptr);
  }
}

// Sum of the nS fp32 partials (already in dW2's and dW1's layouts), four elements per thread
// per array; the sum runs in split order, so it is deterministic.
template <bool BF16>
__global__ void __launch_bounds__(256)
dw_reduce_kernel(const float* __restrict__ ws, void* __restrict__ dW1, void* __restrict__ dW2, int H, int E, int D,
                 int nS, int outf32) {
  const size_t per = (size_t)H * E * D;  // a multiple of 8 (E % 8 == 0)
  const size_t n4 = per / 4;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q < 2 * n4; q += stride) {
    const bool second = q >= n4;  // 0: dW2 slices, 1: dW1 slices
    const size_t i = (second ? q - n4 : q) * 4;
    const float* src = ws + (second ? (size_t)nS * per : 0) + i;
    float4 acc = *(const float4*)src;
    for (int s = 1; s < nS; ++s) {
      const float4 v = *(const float4*)(src + (size_t)s * per);
      acc.x += v.x;
      acc.y += v.y;
      acc.z += v.z;
      acc.w += v.w;
    }
    void* dst = second ? dW1 : dW2;
    if (outf32) {
      *(float4*)((float*)dst + i) = acc;
    } else {
      const u32x2 v = {pack2<BF16>(acc.x, acc.y), pack2<BF16>(acc.z, acc.w)};
      *(u32x2*)((u16*)dst + i) = v;
    }
  }
}

// ------------------------------------------------------------------------------------
// dX from the stored dZ (dxg_kernel): dX = dZ W1^T per head, a GEMM over E, when the dW
// programs store dZ (the io-dtype value the reference's dX product takes,
// flashmlp.py:227-235) instead of the dX programs recomputing Z and dH. A tile is TP blocks of
// 256 rows of one head (a block is one contiguous run of dZ, chunk after chunk), 8 waves x 32
// rows of each block; per 32-column
// E-chunk c a wave issues D/16 MFMAs dX^T += W1c(c) dZ(c)^T (the transposed product: each lane
// ends with whole row pieces of dX; a lane swap makes each bf16/fp16 store 16 bytes).
// Persistent: one workgroup per CU walks its tiles as one stream of (tile, chunk) steps, so
// the loads run ahead across tile boundaries and no tile pays the memory latency up front.
// LDS: a ring of dZ chunks (per 256-row block 8 sub-blocks [32 e][32 positions], 64-byte rows;
// sub-block w = wave w's rows, read with ds_read_b64_tr_b16 like a row-major [e][b] tile)
// streamed from HBM (TP = 1: 8 slots 7 steps ahead), and a ring of W1c chunks ([D][32],
// 64-byte rows, 16-byte chunk q of row r at q ^ ((r >> 2) & 3), read row-wise; L2-resident)
// 3 steps ahead. One barrier per step.
// Stored positions are sig-permuted within 16 rows: the lane holding position m holds row sig(m).
// ------------------------------------------------------------------------------------
// TP = 2 (the default): a tile is two consecutive 256-row blocks of one head, so each W1c chunk
// (and each W1c operand read from LDS) serves both: half the W1c traffic, which a copy of the
// kernel with no W1c traffic priced at 33 us of the cfg4 backward; a step then loads two 16 KB
// dZ chunks into a 32 KB slot of a 4-slot ring three steps ahead, and a wave keeps two
// accumulator sets (190 VGPRs at D = 128). Measured at cfg4: backward 787 -> 763 us, step
// +1.7 % (same box, 3 rounds each).
__host__ __device__ constexpr int dxg_zs(int TP) { return TP == 1 ? 8 : 4; }  // dZ ring slots (TP x 16 KB each)
__host__ __device__ constexpr int dxg_zpf(int TP) { return dxg_zs(TP) - 1; }  // step j + ZPF reuses the slot of step j - 1
constexpr int DXG_ZS = dxg_zs(1);
constexpr int DXG_WS = 4;  // W1c ring slots (64 D bytes each)
constexpr int DXG_WPF = 3;
static_assert(DXG_WPF <= DXG_WS - 1 && DXG_WPF <= dxg_zpf(2), "rings");

template <bool BF16, int D, int TP = 1>
__global__ void __launch_bounds__(DX2_NT) __attribute__((amdgpu_waves_per_eu(2, 2)))
dxg_kernel(const u16* __restrict__ dzt, const u16* __restrict__ W1, void* __restrict__ dX, int B, int Bp, int E,
           int Ep, int tiles_per_head, int n_tiles, int outf32) {
  static_assert(TP == 1 || TP == 2, "256-row blocks per tile");
  constexpr int NTN = D / 32;
  constexpr int ZT = 32 * 256 * 2;      // dZ chunk bytes of one 256-row block
  constexpr int ZS = dxg_zs(TP), ZPF = dxg_zpf(TP);
  constexpr int ZTS = TP * ZT;          // dZ slot bytes
  constexpr int WOFF = ZS * ZTS;        // W1c ring after the dZ ring
  constexpr int WT = 64 * D;            // W1c chunk bytes
  constexpr int NZ = ZT / 16 / DX2_NT;  // dZ pieces per lane per block chunk (2)
  constexpr int W1W = D / 16;           // waves whose lanes cover W1c's 4 D pieces once (the rest repeat them)
  static_assert(NZ * 16 * DX2_NT == ZT, "dZ pieces");
  const int nblk = Bp / DX2_ROWS;       // 256-row blocks per head

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = lane >> 4, i16 = lane & 15, g = lane >> 5, l32 = lane & 31;
  const int NC = (E + 31) >> 5;
  const int nwg = (int)gridDim.x, wg = (int)blockIdx.x;
  const int my_tiles = wg < n_tiles ? (n_tiles - 1 - wg) / nwg + 1 : 0;
  const int steps = my_tiles * NC;
  // tile k of this workgroup: virtual index v = k * nwg + wg, taken in descending row order over
  // all heads (v = 0 .. H - 1 are the last tiles of heads 0 .. H - 1). The dW programs
  // walk their rows upwards, so the dZ they stored last is read first, while the device's
  // memory-side cache still holds it (measured at cfg4: 288 -> 270 us). When nwg is a multiple
  // of H (cfg4: 256 and 32), workgroup wg serves head wg mod H only, on XCD wg mod 8 (the
  // dispatch order), so each XCD's L2 holds the W1 of H / 8 heads.
  const int n_heads = n_tiles / tiles_per_head;
  auto tile_of = [&](int k) {
    const int v = k * nwg + wg;
    const int h = v % n_heads, bt = tiles_per_head - 1 - v / n_heads;
    return h * tiles_per_head + bt;
  };

  // dZ piece p = k * 512 + 64 wave + lane: the chunk is stored as its LDS image, 16 p either way
  unsigned zOff[NZ];
#pragma unroll
  for (int k = 0; k < NZ; ++k) zOff[k] = (unsigned)(k * DX2_NT + wave * 64 + lane) * 16u;
  // W1c piece p = 64 (wave % W1W) + lane: row r = p / 4, logical chunk q = (p % 4) ^ ((r / 4) % 4)
  const unsigned pw = (unsigned)(wave % W1W) * 64u + lane;
  const unsigned wr = pw >> 2, wq = (pw & 3u) ^ ((wr >> 2) & 3u);
  const unsigned wOff = wr * (unsigned)E * 2u + wq * 16u;
  const int wCol = (int)(wq * 8u);

  // step j = (tile k, chunk c) of this workgroup; steps past the last load nothing (zero-size
  // resources), so every step issues the same number of loads and the vmcnt waits stay exact.
  // Each request stream keeps its own cursor; the tile's addresses change only between tiles.
  struct Cursor {
    int j, k, c, nb;
    const u16* z;  // dZ chunk c of tile k's first block
    const u16* w;  // W1 columns 32 c .. of tile k's head
  };
  auto seek = [&](Cursor& q) {  // q.k changed: the new tile's base addresses
    const int t = q.k < my_tiles ? tile_of(q.k) : 0;
    const int h = t / tiles_per_head, bt = t - h * tiles_per_head;
    // the tile's blocks' chunks, 8192 elements each, block after block
    q.z = dzt + ((size_t)h * Bp + (size_t)bt * TP * DX2_ROWS) * Ep;
    q.w = W1 + (size_t)h * D * E;
    q.nb = min(TP, nblk - bt * TP);  // blocks of the tile within the head (TP = 2: the last may hold one)
  };
  auto advance = [&](Cursor& q) {
    ++q.j;
    if (++q.c == NC) {
      q.c = 0;
      ++q.k;
      seek(q);
    } else {
      q.z += 32 * 256;
      q.w += 32;
    }
  };
  auto dma_z = [&](const Cursor& q) {
#pragma unroll
    for (int tp = 0; tp < TP; ++tp) {
      const i32x4 rz = make_rsrc_words(q.z + (size_t)tp * DX2_ROWS * Ep, q.k < my_tiles && tp < q.nb ? ZT : 0);
      const int base = (q.j & (ZS - 1)) * ZTS + tp * ZT;
#pragma unroll
      // the one read of each dZ block: non-temporal (step +0.5-1 % at cfg4 over cached loads)
      for (int i = 0; i < NZ; ++i) buf_load16_lds_nt(rz, zOff[i], base + (i * DX2_NT + wave * 64) * 16);
    }
  };
  auto dma_w = [&](const Cursor& q) {
    const int lim = E - q.c * 32;
    const int rem = D * E * 2 - 64 * q.c;
    const i32x4 rw = make_rsrc_words(q.w, q.k < my_tiles && rem > 0 ? rem : 0);
    buf_load16_lds(rw, wCol < lim ? wOff : BUF_OOB, WOFF + (q.j & (DXG_WS - 1)) * WT + (wave % W1W) * 1024);
  };

  // A operand (dZ, rows = this wave's 32 positions, k = 16 s + 8 g + j): two transposed reads
  // of block `wave`; B operand (W1c row 32 nt + l32, piece 2 s + g)
  const int laneA = wave * 2048 + (8 * g + (i16 >> 2)) * 64 + 32 * (G & 1) + 8 * (i16 & 3);
  int offB[2];
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2) offB[s2] = WOFF + l32 * 64 + (((2 * s2 + g) ^ ((l32 >> 2) & 3)) << 4);

  f32x16 acc[TP][NTN];
#pragma unroll
  for (int tp = 0; tp < TP; ++tp)
#pragma unroll
    for (int nt = 0; nt < NTN; ++nt) acc[tp][nt] = zero16();

  // step i requests dZ of step i + ZPF, then W1c of step i + DXG_WPF; the prologue runs the
  // same order for i < 0, so at step j the loads issued after W1c(j) are those of steps
  // j - 2 .. j - 1 (DXG_WPF - 1 of them)
  Cursor qz{0, 0, 0, 0, nullptr, nullptr};
  seek(qz);
  Cursor qw = qz;
#pragma unroll
  for (int i = -ZPF; i < 0; ++i) {
    dma_z(qz);
    advance(qz);
    if (i + DXG_WPF >= 0) {
      dma_w(qw);
      advance(qw);
    }
  }
  int c = 0, k = 0;  // chunk and tile of step j
  int since = 1 << 20;  // steps since the last tile end
  for (int j = 0; j < steps; ++j) {
    // this wave's pieces of step j (dZ and W1c) have landed: the loads of steps j - 2, j - 1 may
    // stay in flight and, when a tile ended in steps j - 3 .. j - 1 (one at most when NC >= 3),
    // that tile's stores, issued after W1c(j) (vmcnt counts loads and stores in issue order)
    constexpr int NW0 = (TP * NZ + 1) * (DXG_WPF - 1);
    if (++since <= DXG_WPF && NC >= DXG_WPF) {
      if (outf32) wait_vmcnt<NW0 + TP * 4 * NTN>();
      else wait_vmcnt<NW0 + TP * 2 * NTN>();
    } else {
      wait_vmcnt<NW0>();
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();  // step j visible; step j - 1 no longer read
    asm volatile("" ::: "memory");
    dma_z(qz);
    advance(qz);
    dma_w(qw);
    advance(qw);
    const int zb = (j & (ZS - 1)) * ZTS, wb = (j & (DXG_WS - 1)) * WT;
    u32x4 a[TP][2], b[2][NTN];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
#pragma unroll
      for (int tp = 0; tp < TP; ++tp)
        a[tp][s2] = cat(lds_read_tr(zb + tp * ZT + laneA + s2 * 1024), lds_read_tr(zb + tp * ZT + laneA + s2 * 1024 + 256));
#pragma unroll
      for (int nt = 0; nt < NTN; ++nt) b[s2][nt] = lds_read16(wb + offB[s2] + nt * 2048);
    }
    // dX^T tile nt = W1c rows 32 nt .. (A) times the dZ positions (B): C layout lane = position
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int tp = 0; tp < TP; ++tp)
#pragma unroll
        for (int nt = 0; nt < NTN; ++nt) acc[tp][nt] = mfma<BF16>(b[s2][nt], a[tp][s2], acc[tp][nt]);
    if (++c == NC) {  // tile done: lane l32 holds row sig(l32) of the wave's 32 in each block,
                      // columns 32 nt + 8 q + 4 g + 0..3 in acc[tp][nt][4 q .. 4 q + 3]: 16-byte
                      // buffer stores, rows past B out of range
      const int t = tile_of(k);  // once per tile
      const int h = t / tiles_per_head, bt = t - h * tiles_per_head;
      const unsigned r = (unsigned)(wave * 32) + sig((unsigned)l32);
#pragma unroll
      for (int tp = 0; tp < TP; ++tp) {
        const int blk = bt * TP + tp;
        const int rows = clamp0(B - blk * DX2_ROWS, DX2_ROWS);
        if (outf32) {
          const Rsrc ro = make_rsrc((const float*)dX + ((size_t)h * B + (size_t)blk * DX2_ROWS) * D, rows * D * 4);
#pragma unroll
          for (int nt = 0; nt < NTN; ++nt)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const u32x4 v = {__float_as_uint(acc[tp][nt][4 * q]), __float_as_uint(acc[tp][nt][4 * q + 1]),
                               __float_as_uint(acc[tp][nt][4 * q + 2]), __float_as_uint(acc[tp][nt][4 * q + 3])};
              __builtin_amdgcn_raw_buffer_store_b128(v, ro, (int)((r * D + 32 * nt + 8 * q + 4 * g) * 4u), 0, 0);
            }
        } else {
          const Rsrc ro = make_rsrc((const u16*)dX + ((size_t)h * B + (size_t)blk * DX2_ROWS) * D, rows * D * 2);
#pragma unroll
          for (int nt = 0; nt < NTN; ++nt) {
            u32x2 v[4];
#pragma unroll
            for (int q = 0; q < 4; ++q)
              v[q] = u32x2{pack2<BF16>(acc[tp][nt][4 * q], acc[tp][nt][4 * q + 1]),
                           pack2<BF16>(acc[tp][nt][4 * q + 2], acc[tp][nt][4 * q + 3])};
#pragma unroll
            for (int p = 0; p < 2; ++p) {
              // lanes 0-31 hold columns 8q + 0..3, lanes 32-63 8q + 4..7: one swap gives lane g
              // columns 16 p + 8 g .. + 7
              const auto s0 = __builtin_amdgcn_permlane32_swap(v[2 * p][0], v[2 * p + 1][0], false, false);
              const auto s1 = __builtin_amdgcn_permlane32_swap(v[2 * p][1], v[2 * p + 1][1], false, false);
              const u32x4 w = {s0[0], s1[0], s0[1], s1[1]};
              __builtin_amdgcn_raw_buffer_store_b128(w, ro, (int)((r * D + 32 * nt + 16 * p + 8 * g) * 2u), 0, 0);
            }
          }
        }
      }
      since = 0;
#pragma unroll
      for (int tp = 0; tp < TP; ++tp)
#pragma unroll
        for (int nt = 0; nt < NTN; ++nt) acc[tp][nt] = zero16();
      c = 0;
      ++k;
    }
  }
  wait_vmcnt<0>();  // loads past the last step are still landing
}

// ------------------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------------------
// ------------------------------------------------------------------------------------
// Backward plan. The single launch runs H nE nS dW programs and H ceil(B / 256) dX programs,
// one per CU at a time, one role after the other in workgroup order. The B split nS and the
// order come from an estimate of the launch's makespan:
//   * a program costs a fixed part plus its work at a per-CU rate, the work counted in MAC
//     equivalents per element of the (rows x E) activation plane: 4 D MACs (6 D with the hi/lo
//     dW terms) plus the activation's VALU share for a dW program, 3 D plus the activation's
//     share for a dX program;
//   * the first role's programs are dealt round-robin, each later program goes to the CU that
//     frees first (list scheduling);
//   * nS > 1 adds the partial reduction (a launch plus its fp32 traffic).
// Constants fitted to MI355X timings of 14 shapes x activations x (order, nS); the choice the
// estimate makes is within 2.5 % of the best measured one for each of them.
// ------------------------------------------------------------------------------------
namespace {

constexpr double kPlanFixedUs = 3.0;      // per program
constexpr double kPlanRate = 4.5e6;       // MAC equivalents per microsecond per CU
constexpr double kPlanValuMacs = 20.0;    // MAC equivalents per VALU instruction per element
constexpr double kPlanHbmBytesPerUs = 5.0e6;
constexpr double kPlanLaunchUs = 4.0;
constexpr double kPlanDzBytesPerUs = 4.9e6;  // stored-dZ form: dZ bytes per time unit (store + reload)
constexpr double kPlanDzFixedUs = 5.0;

// VALU instructions per element of the activation plane (dX role: act'; dW role: act and act')
double valu_dx(int act) { return act == ACT_SILU ? 8.5 : act == ACT_SIGMOID ? 6.5 : act == ACT_LEAKY ? 3.0 : 1.0; }
double valu_dw(int act) { return act == ACT_SILU ? 9.0 : act == ACT_SIGMOID ? 7.0 : act == ACT_LEAKY ? 4.0 : 1.5; }

// Completion time of n1 programs of t1 dealt round-robin over N CUs, followed by n2 programs of
// t2 each started on the first CU to come free. The n2 programs take the n2 earliest of the
// start slots low + k t2 (the CUs done with the first role at `low`) and high + k t2 (the
// others); the n2-th slot is found by bisection on the slot count.
double list_makespan(long long n1, double t1, long long n2, double t2, long long N) {
  const long long q = n1 / N, r = n1 % N;
  const double low = (double)q * t1, high = r ? (double)(q + 1) * t1 : low;
  const double end1 = n1 > 0 ? high : 0.0;
  if (n2 <= 0) return end1;
  const double a = (double)(N - r), b = (double)r;
  auto slots_by = [&](double T) {
    double c = 0.0;
    if (T >= low) c += a * (std::floor((T - low) / t2) + 1.0);
    if (b > 0 && T >= high) c += b * (std::floor((T - high) / t2) + 1.0);
    return c;
  };
  double lo = low, hi = high + (double)n2 * t2;
  for (int it = 0; it < 64; ++it) {
    const double mid = 0.5 * (lo + hi);
    if (slots_by(mid) >= (double)n2) hi = mid;
    else lo = mid;
  }
  return std::max(end1, hi + t2);
}

long long rows_for_split(long long B, long long ns) {
  long long rps = (B + ns - 1) / ns;
  rps = (rps + DW_BT - 1) / DW_BT * DW_BT;
  return rps < DW_BT ? (long long)DW_BT : rps;
}

BwdPlan make_plan(int64_t H, int64_t B, int64_t D, int64_t E, int act, bool hilo, int dz_mode, int num_cus,
                  size_t max_ws) {
  // Everything that decides how dX is computed (the stored-dZ form or not, the dX programs' E
  // split, the split of the ragged dX tiles) follows the default dW mode's plan, so dX does not
  // depend on the dW mode (FMLP_DW_HILO changes only dW).
  int fixed_des = 0, fixed_dxs = -1, fixed_dz = -1;
  if (hilo) {
    const BwdPlan d = make_plan(H, B, D, E, act, false, dz_mode, num_cus, max_ws);
    fixed_dz = d.dz ? 1 : 0;
    if (!d.dz) {
      fixed_des = d.dx_es;
      fixed_dxs = d.dxs_xs > 0 ? 1 : 0;
    } else {  // used only if the stored-dZ form does not fit this mode's workspace limit
      const BwdPlan r = make_plan(H, B, D, E, act, false, DZ_NEVER, num_cus, max_ws);
      fixed_des = r.dx_es;
      fixed_dxs = r.dxs_xs > 0 ? 1 : 0;
    }
  }
  BwdPlan p{};
  const long long N = num_cus > 0 ? num_cus : 1;
  // dW programs of ET E-columns: 128, or at D = 64 with the dX programs' E split also 64 (twice
  // the programs, each half the work, for grids that leave CUs idle); FMLP_BWD_ET (read once per
  // process) forces 128 or 64 where allowed
  static const int et_env = env_int("FMLP_BWD_ET", 0);
  auto nE_for = [&](long long et) { return (E + et - 1) / et; };
  const long long base = H * nE_for(DW_ET);  // the stored-dZ form's dW programs (128 columns)
  auto ws_for = [&](long long ns) { return ns > 1 ? (size_t)2 * ns * H * E * D * sizeof(float) : (size_t)0; };
  // dX programs of 256 rows, or at D = 64 of 128 rows with E in two parts (half the time each)
  auto n_dx_for = [&](int des) { return H * ((B + DX2_ROWS / des - 1) / (DX2_ROWS / des)); };
  auto tx_for = [&](int des) {
    return kPlanFixedUs + (double)(DX2_ROWS / des) * E * (3.0 * D + valu_dx(act) * kPlanValuMacs) / kPlanRate;
  };
  const int max_des = D == 64 ? 2 : 1;
  auto w_per_row_for = [&](long long et) {
    return (double)et * ((hilo ? 6.0 : 4.0) * D + valu_dw(act) * kPlanValuMacs) / kPlanRate;
  };
  const double w_per_row = w_per_row_for(DW_ET);
  // candidates nS = 1, 2, 4, ... up to B / 256 and two dW programs per CU (which keeps the fp32
  // partials within 64 MiB at D <= 128 on 256 CUs), whose workspace fits max_ws
  const long long max_ns = B / 256 > 1 ? B / 256 : 1;
  auto cap_for = [&](long long nprog) {
    long long c = nprog > 0 ? 2 * N / nprog : 1;
    if (c < 1) c = 1;
    if (c > max_ns) c = max_ns;
    return c;
  };
  const long long cap = cap_for(base);
  // FMLP_BWD_NS / FMLP_BWD_ORDER (read once per process) force the split and the order
  // (1: dW programs first, 2: dX programs first)
  static const int ns_env = env_int("FMLP_BWD_NS", 0);
  static const int order_env = env_int("FMLP_BWD_ORDER", 0);
  // FMLP_BWD_DXES (read once per process) forces the dX programs' E split (1 or 2, D = 64)
  static const int des_env = env_int("FMLP_BWD_DXES", 0);
  // Ragged last dX tiles (B not a multiple of the dX rows): one per head, each a whole program
  // for a few rows, which can leave a last round of H programs on an otherwise idle device. The
  // plan may split them over E into xs parts of at least 4 chunks (fp32 partials in the
  // workspace, summed by a second launch); FMLP_BWD_DXSPLIT=0 (read once per process) never does.
  static const int dxs_env = env_int("FMLP_BWD_DXSPLIT", -1);
  const long long nch = (E + 31) / 32;
  long long dxs_xs = std::min<long long>(16, nch / 4);
  const long long dxs_nct = dxs_xs >= 2 ? (nch + dxs_xs - 1) / dxs_xs : nch;
  if (dxs_xs >= 2) dxs_xs = (nch + dxs_nct - 1) / dxs_nct;
  auto dxs_bytes = [&](int des) { return (size_t)H * dxs_xs * (DX2_ROWS / des) * D * sizeof(float); };
  double best_t = 0.0;
  long long best_ns = 1;
  bool best_dx_first = false, best_dxs = false;
  int best_des = 1, best_et = DW_ET;
  for (int des = 1; des <= max_des; ++des) {
    if (des_env > 0 && des != des_env) continue;
    if (fixed_des > 0 && des != fixed_des) continue;
    const long long n_dx = n_dx_for(des), T_dx = n_dx / (H > 0 ? H : 1);
    const double tx = tx_for(des);
    const bool rag = B % (DX2_ROWS / des) != 0 && T_dx >= 2 && dxs_xs >= 2 && dxs_env != 0 && fixed_dxs != 0;
    for (int et = DW_ET; et >= 64; et /= 2) {
      if (et != DW_ET && !(D == 64 && des == 2)) continue;
      if (et_env > 0 && et != et_env && (et_env == DW_ET || (D == 64 && des == 2))) continue;
      const long long base_et = H * nE_for(et), cap_et = cap_for(base_et);
      const double wrow = w_per_row_for(et);
      for (long long ns = 1; ns <= (ns_env > 0 ? 1 : cap_et); ns *= 2) {
        const long long want = ns_env > 0 ? (ns_env < max_ns ? ns_env : max_ns) : ns;
        const long long rps = rows_for_split(B, want), eff = B > rps ? (B + rps - 1) / rps : 1;
        if (eff > 1 && ws_for(eff) > max_ws) break;
        const double tw = kPlanFixedUs + (double)rps * wrow;
        const long long n_dw = base_et * eff;
        const double red = eff > 1 ? kPlanLaunchUs + (double)(2 * eff + 1) * H * E * D * 4.0 / kPlanHbmBytesPerUs : 0.0;
        const bool dxs_fits = rag && (ws_for(eff) + 255) / 256 * 256 + dxs_bytes(des) <= max_ws;
        for (int split = 0; split <= 1; ++split) {
          if (split ? !dxs_fits : fixed_dxs == 1 && dxs_fits) continue;
          // the split tiles' parts are the launch's last workgroups: they fill the time CUs
          // spend idle before the last of the other programs ends (idle time only comes at the
          // end of a list schedule), what does not fit there takes a last partial round of at
          // least one part; then the launch that sums them
          const long long nx = split ? n_dx - H : n_dx;
          const double tp = kPlanFixedUs + (tx - kPlanFixedUs) / dxs_xs, wp = (double)H * dxs_xs * tp;
          for (int o = 1; o <= 2; ++o) {
            if (order_env && o != order_env) continue;
            const double t2 = o == 1 ? list_makespan(n_dw, tw, nx, tx, N) : list_makespan(nx, tx, n_dw, tw, N);
            double t = t2 + red;
            if (split) {
              const double idle = (double)N * t2 - ((double)n_dw * tw + (double)nx * tx);
              const double over = wp - std::max(0.0, idle);
              if (over > 0.0) t += std::max(over / (double)N, tp);
              t += kPlanLaunchUs;
            }
            if (best_t == 0.0 || t < best_t) {
              best_t = t;
              best_ns = eff;
              best_dx_first = o == 2;
              best_des = des;
              best_dxs = split == 1;
              best_et = et;
            }
          }
        }
      }
    }
  }
  p.et_w = best_et;
  p.dx_es = best_des;
  p.dx_tiles_per_head = (int)((B + DX2_ROWS / best_des - 1) / (DX2_ROWS / best_des));
  p.n_dx = (long long)p.dx_tiles_per_head * H;
  if (best_dxs) {
    p.dxs_xs = (int)dxs_xs;
    p.dxs_nct = (int)dxs_nct;
    p.n_dx -= H;
  }
  // Stored-dZ form: the dW launch alone (programs dealt over the CUs) and its reduction, then
  // storing dZ and streaming it back through the dX GEMM (memory-bound: a rate per byte, in the
  // same time units, and a fixed part for the extra launch). Fitted to the same-box times of
  // cfg2-cfg5 in both forms. FMLP_BWD_DZ (read once per process): 0 never, 1 whenever the
  // workspace allows it, unset: when the estimate is lower (dz_mode overrides it, per call).
  static const int dz_env = env_int("FMLP_BWD_DZ", -1);
  const int dz_want = dz_mode != DZ_AUTO ? (dz_mode == DZ_FORCE ? 1 : 0) : dz_env;
  const long long Bp = (B + DX2_ROWS - 1) / DX2_ROWS * DX2_ROWS;
  const size_t dz_head = (size_t)nE_for(DW_ET) * DW_ET * (size_t)Bp * 2u;
  double best_dz = 0.0;
  long long best_dz_ns = 1;
  if (dz_want != 0 && B > 0 && dz_head < ((size_t)1 << 31)) {
    const double t_dx = kPlanDzFixedUs + (double)H * dz_head / kPlanDzBytesPerUs;
    for (long long ns = 1; ns <= (ns_env > 0 ? 1 : cap); ns *= 2) {
      const long long want = ns_env > 0 ? (ns_env < max_ns ? ns_env : max_ns) : ns;
      const long long rps = rows_for_split(B, want), eff = B > rps ? (B + rps - 1) / rps : 1;
      const size_t need = (ws_for(eff) + 255) / 256 * 256 + (size_t)H * dz_head;
      if (need > max_ws) break;
      const double tw = kPlanFixedUs + (double)rps * w_per_row;
      const double red = eff > 1 ? kPlanLaunchUs + (double)(2 * eff + 1) * H * E * D * 4.0 / kPlanHbmBytesPerUs : 0.0;
      const double t = list_makespan(base * eff, tw, 0, 0.0, N) + red + t_dx;
      if (best_dz == 0.0 || t < best_dz) {
        best_dz = t;
        best_dz_ns = eff;
      }
    }
  }
  p.dz = best_dz > 0.0 && (fixed_dz >= 0 ? fixed_dz == 1 : (dz_want == 1 || best_dz < best_t));
  if (p.dz) {
    best_ns = best_dz_ns;
    best_dx_first = false;
    p.dx_es = 1;
    p.dx_tiles_per_head = (int)((B + DX2_ROWS - 1) / DX2_ROWS);
    p.dxs_xs = 0;
    p.dxs_nct = 0;
    p.et_w = DW_ET;
  }
  p.nE = (int)nE_for(p.et_w);
  const long long rps = rows_for_split(B, best_ns);
  p.nS = (int)(B > rps ? (B + rps - 1) / rps : 1);
  p.rows_per_split = (int)rps;
  p.n_dw = H * (long long)p.nE * p.nS;
  p.dx_first = best_dx_first;
  p.ws_bytes = ws_for(p.nS);
  p.dw_ws_bytes = p.ws_bytes;
  if (p.dxs_xs > 0) {  // the split dX tiles' partials after the dW partials
    p.n_dxs = H * (long long)p.dxs_xs;
    p.dxs_off = (p.ws_bytes + 255) / 256 * 256;
    p.ws_bytes = p.dxs_off + dxs_bytes(p.dx_es);
  }
  if (p.dz) {
    p.Bp = (int)Bp;
    p.dz_off = (p.ws_bytes + 255) / 256 * 256;
    p.ws_bytes = p.dz_off + (size_t)H * dz_head;
    p.n_dx = H * (Bp / DX2_ROWS);
    // dxg_kernel is persistent: one workgroup per CU (a multiple of 8, the XCD count), at most
    // one per tile
    p.n_xg = (int)std::min<long long>(p.n_dx, std::max<long long>(8, N / 8 * 8));
  }
  return p;
}

}  // namespace

// Plans are computed once per distinct call shape (a small cache of recent ones).
BwdPlan plan_bwd(int64_t H, int64_t B, int64_t D, int64_t E, int act, bool hilo, int dz_mode, int num_cus,
                 size_t max_ws) {
  struct Entry {
    int64_t H, B, D, E;
    int act, hilo, dz, cus;
    size_t max_ws;
    BwdPlan plan;
  };
  static std::mutex mu;
  static Entry cache[16];
  static int used = 0, next = 0;
  {
    std::lock_guard<std::mutex> lock(mu);
    for (int i = 0; i < used; ++i) {
      const Entry& c = cache[i];
      if (c.H == H && c.B == B && c.D == D && c.E == E && c.act == act && c.hilo == (int)hilo &&
          c.dz == dz_mode && c.cus == num_cus && c.max_ws == max_ws)
        return c.plan;
    }
  }
  const BwdPlan p = make_plan(H, B, D, E, act, hilo, dz_mode, num_cus, max_ws);
  std::lock_guard<std::mutex> lock(mu);
  cache[next] = Entry{H, B, D, E, act, (int)hilo, dz_mode, num_cus, max_ws, p};
  next = (next + 1) % 16;
  if (used < 16) ++used;
  return p;
}

// B split of the D = 256 dW programs: the nS (1, 2, 4, ...) with the least estimated time,
// rounds of programs over the CUs times a program's time (a fixed part and one per 32-row
// subtile) plus, for nS > 1, the summing launch and the partials' traffic (written, then read).
// FMLP_DW256_NS (read once per process) forces nS where its workspace fits.
Dw256Plan plan_dw256(int64_t H, int64_t B, int64_t E, bool hilo, int num_cus, size_t max_ws) {
  constexpr double kFixedUs = 4.0, kSubUs = 1.0, kSubHiloUs = 1.4;
  static const int ns_env = env_int("FMLP_DW256_NS", 0);
  Dw256Plan p{};
  p.nE = (int)((E + DW_ET - 1) / DW_ET);
  p.nS = 1;
  p.rows_per_split = (int)rows_for_split(B, 1);
  p.n = H * p.nE;
  p.ws_bytes = 0;
  if (p.n <= 0 || B <= 0) return p;
  const long long N = num_cus > 0 ? num_cus : 1;
  const long long max_ns = B / 256 > 1 ? B / 256 : 1;
  const double t_sub = hilo ? kSubHiloUs : kSubUs;
  double best = 1e300;
  for (long long ns = 1; ns <= max_ns; ns *= 2) {
    const long long rps = rows_for_split(B, ns), eff = (B + rps - 1) / rps;
    const size_t ws = eff > 1 ? (size_t)2 * eff * H * E * 256 * sizeof(float) : 0;
    if (ws > max_ws) continue;
    const long long progs = H * p.nE * eff, rounds = (progs + N - 1) / N;
    double cost = (double)rounds * (kFixedUs + (double)(rps / DW_BT) * t_sub);
    if (eff > 1) cost += kPlanLaunchUs + 2.0 * (double)ws / kPlanHbmBytesPerUs;
    // with the override: the first split that fits, replaced by the forced one
    const bool take = ns_env > 0 ? (eff == ns_env || best == 1e300) : cost < best;
    if (take) {
      best = cost;
      p.nS = (int)eff;
      p.rows_per_split = (int)rps;
      p.n = progs;
      p.ws_bytes = ws;
    }
  }
  return p;
}

// dynamic LDS of the dW role: a 3-group ring of subtiles and the two weight tiles
template <int D, int ET>
constexpr size_t dw_lds_bytes() {
  return 3u * 2u * (DW2_NW / (ET / 32)) * 64u * D + 2u * 2u * ET * D;
}

// sum of the dW programs' fp32 partials when B is split (nS > 1)
template <bool BF16>
static hipError_t launch_dw_reduce(const BwdArgs& a, int nS, hipStream_t st) {
  if (nS <= 1) return hipSuccess;
  const size_t items = 2 * ((size_t)a.H * a.E * a.D / 4);
  size_t blocks = (items + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(dw_reduce_kernel<BF16>, dim3((unsigned)blocks), dim3(256), 0, st, (const float*)a.ws, a.dw1, a.dw2,
                     (int)a.H, (int)a.E, (int)a.D, nS, a.out_f32 ? 1 : 0);
  return hipGetLastError();
}

template <bool BF16, int D, int ACT, int DES, int ET>
static hipError_t launch_bwd_t(const BwdArgs& a, const BwdPlan& p, hipStream_t st) {
  if (p.n_dw + p.n_dx + p.n_dxs > 0x7fffffffLL || (long long)p.dx_tiles_per_head * a.H > 0x7fffffffLL)
    return hipErrorInvalidValue;
  hipError_t e;
  // the dW role's: two weight tiles and three subtile pairs (256 D bytes each); at least the
  // dX role's rings (one or two parts of DX_NSLOT slots of 128 D bytes)
  constexpr size_t lds = std::max<size_t>(dw_lds_bytes<D, ET>(), (size_t)DES * DX_NSLOT * 128u * D);
  static_assert(dw_lds_bytes<D, DW_ET>() == 1280u * D, "the 128-column form's LDS");
  auto reduce = [&]() { return launch_dw_reduce<BF16>(a, p.nS, st); };
  if (p.dz && a.want_dx && a.want_dw) {  // stored-dZ form: dW programs storing dZ, their reduction, then the dX GEMM
    u16* dzt = (u16*)((char*)a.ws + p.dz_off);
    const int Ep = p.nE * DW_ET;
    auto launch_w = [&](auto k) {
      static std::atomic<unsigned long long> lds_set{0};
      hipError_t r = set_lds_once((const void*)k, (int)lds, lds_set);
      if (r != hipSuccess) return r;
      hipLaunchKernelGGL(k, dim3((unsigned)p.n_dw), dim3(DW2_NT), lds, st, (const u16*)a.x, (const u16*)a.w1,
                         (const u16*)a.w2, (const u16*)a.dout, a.dw1, a.dw2, (float*)a.ws, (int)a.H, (int)a.B,
                         (int)a.E, p.nE, p.nS, p.rows_per_split, a.out_f32 ? 1 : 0, dzt, p.Bp);
      return hipGetLastError();
    };
    e = a.dw_hilo ? launch_w(dw2_kernel<BF16, D, ACT, true, true>) : launch_w(dw2_kernel<BF16, D, ACT, false, true>);
    if (e != hipSuccess) return e;
    if ((e = reduce()) != hipSuccess) return e;
    // FMLP_DXG_TP (read once per process): 256-row blocks per dX GEMM tile, 2 (default) or 1
    static const int tp_env = env_int("FMLP_DXG_TP", 2);
    auto launch_g = [&](auto kg, int TP) {
      static std::atomic<unsigned long long> lds_g_set[2] = {};
      const size_t lds_g = (size_t)dxg_zs(TP) * TP * (32 * 256 * 2) + (size_t)DXG_WS * 64 * D;
      hipError_t r = set_lds_once((const void*)kg, (int)lds_g, lds_g_set[TP - 1]);
      if (r != hipSuccess) return r;
      const int tph = (p.Bp / DX2_ROWS + TP - 1) / TP;  // tiles per head
      const long long n_t = a.H * (long long)tph;
      const long long grid = TP == 1 ? p.n_xg : std::min<long long>(n_t, p.n_xg);
      hipLaunchKernelGGL(kg, dim3((unsigned)grid), dim3(DX2_NT), lds_g, st, (const u16*)dzt, (const u16*)a.w1, a.dx,
                         (int)a.B, p.Bp, (int)a.E, Ep, tph, (int)n_t, a.out_f32 ? 1 : 0);
      return hipGetLastError();
    };
    return tp_env == 1 ? launch_g(dxg_kernel<BF16, D, 1>, 1) : launch_g(dxg_kernel<BF16, D, 2>, 2);
  }
  // FMLP_BWD_UNIFIED (read once per process): 1 (default) = one launch holding both roles,
  // 0 = dW programs (and their reduction), then dX programs, as separate launches
  static const int unified = env_int("FMLP_BWD_UNIFIED", 1);
  // a partial backward (FMLP_BWD_NO_DX / FMLP_BWD_NO_DW) launches only the programs it needs;
  // the dX programs alone, where the plan splits the ragged last tiles, are the same launch
  // without dW programs (and the same sum of the parts), so dX is the full call's bit for bit
  const bool both = a.want_dw && p.n_dw > 0 && p.n_dx + p.n_dxs > 0;
  if (unified && a.want_dx && (both || (!a.want_dw && p.n_dxs > 0))) {
    const long long n_dw = a.want_dw ? p.n_dw : 0;
    float* dxs_ws = p.n_dxs > 0 ? (float*)((char*)a.ws + p.dxs_off) : nullptr;
    auto launch_u = [&](auto k) {
      static std::atomic<unsigned long long> lds_set{0};
      hipError_t r = set_lds_once((const void*)k, (int)lds, lds_set);
      if (r != hipSuccess) return r;
      hipLaunchKernelGGL(k, dim3((unsigned)(n_dw + p.n_dx + p.n_dxs)), dim3(DW2_NT), lds, st, (const u16*)a.x,
                         (const u16*)a.w1, (const u16*)a.w2, (const u16*)a.dout, a.dx, a.dw1, a.dw2, (float*)a.ws,
                         (int)a.H, (int)a.B, (int)a.E, p.nE, p.nS, p.rows_per_split, (int)n_dw,
                         p.dx_tiles_per_head, p.dx_first ? 1 : 0, a.out_f32 ? 1 : 0, (int)p.n_dxs, p.dxs_xs,
                         p.dxs_nct, dxs_ws);
      return hipGetLastError();
    };
    e = a.dw_hilo ? launch_u(bwd_kernel<BF16, D, ACT, true, DES, ET>) : launch_u(bwd_kernel<BF16, D, ACT, false, DES, ET>);
    if (e != hipSuccess) return e;
    if (a.want_dw && (e = reduce()) != hipSuccess) return e;
    if (p.n_dxs == 0) return hipSuccess;
    // the ragged dX tiles' partials: split tile s is head s's last tile
    return launch_tile_reduce(dxs_ws, a.dx, BF16, (int)a.B, D, DX2_ROWS / DES, (int)a.H, p.dx_tiles_per_head,
                              p.dxs_xs, (int)a.H, a.out_f32 ? 1 : 0, st);
  }
  if (p.n_dw > 0 && a.want_dw) {
    auto launch_w = [&](auto k) {
      static std::atomic<unsigned long long> lds_set{0};
      hipError_t r = set_lds_once((const void*)k, (int)lds, lds_set);
      if (r != hipSuccess) return r;
      hipLaunchKernelGGL(k, dim3((unsigned)p.n_dw), dim3(DW2_NT), lds, st, (const u16*)a.x, (const u16*)a.w1,
                         (const u16*)a.w2, (const u16*)a.dout, a.dw1, a.dw2, (float*)a.ws, (int)a.H,
                         (int)a.B, (int)a.E, p.nE, p.nS, p.rows_per_split, a.out_f32 ? 1 : 0, (u16*)nullptr, 0);
      return hipGetLastError();
    };
    e = a.dw_hilo ? launch_w(dw2_kernel<BF16, D, ACT, true, false, ET>)
                  : launch_w(dw2_kernel<BF16, D, ACT, false, false, ET>);
    if (e != hipSuccess) return e;
    if ((e = reduce()) != hipSuccess) return e;
  }
  const long long n_dx_all = (long long)p.dx_tiles_per_head * a.H;  // whole tiles only here
  if (n_dx_all > 0 && a.want_dx) {
    const size_t lds_x = (size_t)DES * DX_NSLOT * 128u * D;  // the chunk ring(s)
    auto k = dx2_kernel<BF16, D, ACT, DES>;
    static std::atomic<unsigned long long> lds_set{0};
    e = set_lds_once((const void*)k, (int)lds_x, lds_set);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k, dim3((unsigned)n_dx_all), dim3(DX2_NT), lds_x, st, (const u16*)a.x, (const u16*)a.w1,
                       (const u16*)a.w2, (const u16*)a.dout, a.dx, (int)a.B, (int)a.E, p.dx_tiles_per_head,
                       a.out_f32 ? 1 : 0);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  return hipSuccess;
}

template <bool BF16, int D, int ACT>
static hipError_t launch_bwd_e(const BwdArgs& a, const BwdPlan& p, hipStream_t st) {
  if constexpr (D == 64) {
    if (p.dx_es == 2 && p.et_w == 64) return launch_bwd_t<BF16, D, ACT, 2, 64>(a, p, st);
    if (p.dx_es == 2) return launch_bwd_t<BF16, D, ACT, 2, DW_ET>(a, p, st);
  }
  return launch_bwd_t<BF16, D, ACT, 1, DW_ET>(a, p, st);
}

template <bool BF16, int D>
static hipError_t launch_bwd_a(const BwdArgs& a, const BwdPlan& p, hipStream_t st) {
  switch (a.act) {
    case ACT_SILU: return launch_bwd_e<BF16, D, ACT_SILU>(a, p, st);
    case ACT_LEAKY: return launch_bwd_e<BF16, D, ACT_LEAKY>(a, p, st);
    case ACT_SIGMOID: return launch_bwd_e<BF16, D, ACT_SIGMOID>(a, p, st);
    default: return launch_bwd_e<BF16, D, ACT_NONE>(a, p, st);
  }
}

template <bool BF16, int ACT>
static hipError_t launch_dx256_t(const BwdArgs& a, hipStream_t st) {
  const long long tph = (a.B + 127) / 128, grid = tph * a.H;
  if (grid <= 0) return hipSuccess;
  if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
  constexpr size_t lds = (size_t)dx_nslot(256) * 128u * 256u;
  auto k = dx256_kernel<BF16, ACT>;
  static std::atomic<unsigned long long> lds_set{0};
  hipError_t e = set_lds_once((const void*)k, (int)lds, lds_set);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(256), lds, st, (const u16*)a.x, (const u16*)a.w1, (const u16*)a.w2,
                     (const u16*)a.dout, a.dx, (int)a.B, (int)a.E, (int)tph, a.out_f32 ? 1 : 0);
  return hipGetLastError();
}

template <bool BF16>
static hipError_t launch_dx256_a(const BwdArgs& a, hipStream_t st) {
  switch (a.act) {
    case ACT_SILU: return launch_dx256_t<BF16, ACT_SILU>(a, st);
    case ACT_LEAKY: return launch_dx256_t<BF16, ACT_LEAKY>(a, st);
    case ACT_SIGMOID: return launch_dx256_t<BF16, ACT_SIGMOID>(a, st);
    default: return launch_dx256_t<BF16, ACT_NONE>(a, st);
  }
}

hipError_t launch_dx256(const BwdArgs& a, hipStream_t st) {
  return a.bf16 ? launch_dx256_a<true>(a, st) : launch_dx256_a<false>(a, st);
}

template <bool BF16, int ACT, bool HILO>
static hipError_t launch_dw256_t(const BwdArgs& a, const Dw256Plan& p, hipStream_t st) {
  if (p.n <= 0) return hipSuccess;
  if (p.n > 0x7fffffffLL) return hipErrorInvalidValue;
  constexpr size_t lds = (size_t)DW4_NSLOT * DW4_SLOT;
  auto k = dw256_kernel<BF16, ACT, HILO>;
  static std::atomic<unsigned long long> lds_set{0};
  hipError_t e = set_lds_once((const void*)k, (int)lds, lds_set);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k, dim3((unsigned)p.n), dim3(256), lds, st, (const u16*)a.x, (const u16*)a.w1, (const u16*)a.w2,
                     (const u16*)a.dout, a.dw1, a.dw2, (float*)a.ws, (int)a.H, (int)a.B, (int)a.E, p.nE, p.nS,
                     p.rows_per_split, a.out_f32 ? 1 : 0);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  return launch_dw_reduce<BF16>(a, p.nS, st);
}

template <bool BF16, bool HILO>
static hipError_t launch_dw256_a(const BwdArgs& a, const Dw256Plan& p, hipStream_t st) {
  switch (a.act) {
    case ACT_SILU: return launch_dw256_t<BF16, ACT_SILU, HILO>(a, p, st);
    case ACT_LEAKY: return launch_dw256_t<BF16, ACT_LEAKY, HILO>(a, p, st);
    case ACT_SIGMOID: return launch_dw256_t<BF16, ACT_SIGMOID, HILO>(a, p, st);
    default: return launch_dw256_t<BF16, ACT_NONE, HILO>(a, p, st);
  }
}

hipError_t launch_dw256(const BwdArgs& a, const Dw256Plan& p, hipStream_t st) {
  if (a.bf16) return a.dw_hilo ? launch_dw256_a<true, true>(a, p, st) : launch_dw256_a<true, false>(a, p, st);
  return a.dw_hilo ? launch_dw256_a<false, true>(a, p, st) : launch_dw256_a<false, false>(a, p, st);
}

hipError_t launch_bwd(const BwdArgs& a, const BwdPlan& p, hipStream_t st) {
  if (a.bf16) {
    if (a.D == 128) return launch_bwd_a<true, 128>(a, p, st);
    return launch_bwd_a<true, 64>(a, p, st);
  }
  if (a.D == 128) return launch_bwd_a<false, 128>(a, p, st);
  return launch_bwd_a<false, 64>(a, p, st);
}

}  // namespace fmlp
