// FlashMLP forward kernel for gfx950 (MI355X).
//
// Computes, per head h and B-tile of rows:  O = act(X W1) W2  with fp32 accumulation,
// casting act(Z) to the io dtype before the second contraction (the reference's cast
// point, flashmlp.py:137-150) and O to the io dtype at the store (flashmlp.py:157).
// The (H, B, E) intermediate never leaves registers.
//
// Per workgroup: NW waves, each owning MT 32-row M-tiles (BB = 32*MT*NW rows).
//   * X rows live in registers for the whole kernel, already in the MFMA B-operand layout
//     of Z^T = W1c^T X^T (lane = row b, 8 consecutive d).
//   * E is walked in 32-column chunks. Chunk k's W1c (D x 32) and W2c (32 x D) tiles are
//     staged in an LDS ring of 4 slots; both are read with ds_read_b64_tr_b16, which
//     yields the K-contiguous operands straight from the natural row-major tiles.
//   * Z^T is produced in the MFMA C layout (lane = column b), which is exactly the A
//     operand layout of O += h W2c (lane = row b), so h never round-trips through LDS.
//   * Software pipeline, iteration c:  Z^T(c+1) = W1c(c+1)^T X^T  and  O += h(c-1) W2c(c-1)
//     on the matrix cores while h(c) = act(Z^T(c)) runs on the VALU. The chunk c+2 is
//     prefetched into registers and written to the free slot; one barrier per chunk.
#include "fmlp_device.h"
#include "fmlp_launch.h"
#include <type_traits>

namespace fmlp {

template <bool BF16, int D, int ACT, int NW, int MT>
__global__ void __launch_bounds__(NW * 64)
fwd_kernel(const u16* __restrict__ X, const u16* __restrict__ W1, const u16* __restrict__ W2,
           u16* __restrict__ O, int B, int E, int tiles_per_head) {
  constexpr int NT = NW * 64;          // threads
  constexpr int KS = D / 16;           // K steps of GEMM1
  constexpr int NTN = D / 32;          // N tiles of GEMM2
  constexpr int BB = NW * MT * 32;     // rows per workgroup
  constexpr unsigned SLOT = 128u * D;  // bytes per ring slot: W1c (64*D) + W2c (64*D)
  constexpr unsigned W2OFF = 64u * D;
  constexpr int NP = 8 * D;            // 16-byte pieces per chunk (half W1c, half W2c)
  constexpr int PPT = NP / NT;         // first PPT/2 pieces of a thread are W1c, the rest W2c
  static_assert(NP % (2 * NT) == 0, "pieces per thread");

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int G = lane >> 4, i16 = lane & 15, g = lane >> 5, l32 = lane & 31;
  const int t = xcd_remap(blockIdx.x, gridDim.x);
  const int h = t / tiles_per_head, bt = t - h * tiles_per_head;
  const int NC = (E + 31) >> 5;

  const u16* Xh = X + (size_t)h * B * D;
  const u16* W1h = W1 + (size_t)h * D * E;
  const u16* W2h = W2 + (size_t)h * E * D;
  u16* Oh = O + (size_t)h * B * D;
  const int b_wave = bt * BB + wave * MT * 32;

  // ---- global -> register staging of one chunk, then register -> LDS ----
  u32x4 stg[PPT];
  auto load_chunk = [&](int c) {
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (k < PPT / 2) {  // W1c piece: row d, 8 columns at 8q
        const int p = tid + k * NT;
        const int d = p >> 2, q = p & 3;
        const int e = c * 32 + q * 8;
        if (e < E) v = *(const u32x4*)(W1h + (size_t)d * E + e);
      } else {            // W2c piece: row er, 8 columns at 8q
        const int p = tid + (k - PPT / 2) * NT;
        const int er = p / (D / 8), q = p % (D / 8);
        const int e = c * 32 + er;
        if (e < E) v = *(const u32x4*)(W2h + (size_t)e * D + q * 8);
      }
      stg[k] = v;
    }
  };
  auto store_chunk = [&](int slot) {
    const unsigned base = slot * SLOT;
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
      if (k < PPT / 2) {
        const int p = tid + k * NT;
        const int d = p >> 2, q = p & 3;
        u32x2 lo = {stg[k][0], stg[k][1]}, hi = {stg[k][2], stg[k][3]};
        lds_write8(base + w1c_off(d, 2 * q), lo);
        lds_write8(base + w1c_off(d, 2 * q + 1), hi);
      } else {
        const int p = tid + (k - PPT / 2) * NT;
        const int er = p / (D / 8), q = p % (D / 8);
        lds_write16(base + W2OFF + tile_off<D>(er, q * 8), stg[k]);
      }
    }
  };

  // ---- X rows -> registers (B operand of Z^T = W1c^T X^T) ----
  u32x4 xr[MT][KS];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int b = b_wave + mt * 32 + l32;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (b < B) v = *(const u32x4*)(Xh + (size_t)b * D + ks * 16 + g * 8);
      xr[mt][ks] = v;
    }
  }

  // per-lane LDS offsets (slot-relative)
  // GEMM1 A operand (tr read of W1c): rows 16ks + 8g + 4r + i16/4, unit 4(G%2) + i16%4
  unsigned offA[2][2];
#pragma unroll
  for (int kp = 0; kp < 2; ++kp)
#pragma unroll
    for (int r = 0; r < 2; ++r)
      offA[kp][r] = w1c_off(16 * kp + 8 * g + 4 * r + (i16 >> 2), 4 * (G & 1) + (i16 & 3));
  // GEMM2 B operand (tr read of W2c): rows 16s + 8r + 4g + i16/4, column 32nt + 16(G%2) + 4(i16%4)
  unsigned offB[2][2][NTN];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int nt = 0; nt < NTN; ++nt)
        offB[s][r][nt] = W2OFF + tile_off<D>(16 * s + 8 * r + 4 * g + (i16 >> 2), 32 * nt + 16 * (G & 1) + 4 * (i16 & 3));

  auto gemm1 = [&](int slot, f32x16 (&z)[MT]) {
    const unsigned base = slot * SLOT;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) z[mt] = zero16();
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      // rows advance by 16 per ks: 16 rows * 64 B; the unit swizzle repeats every 32 rows
      const unsigned a0 = base + offA[ks & 1][0] + (ks >> 1) * 2048u;
      const unsigned a1 = base + offA[ks & 1][1] + (ks >> 1) * 2048u;
      const u32x4 A = cat(lds_read_tr(a0), lds_read_tr(a1));
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) z[mt] = mfma<BF16>(A, xr[mt][ks], z[mt]);
    }
  };
  f32x16 o[MT][NTN];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NTN; ++nt) o[mt][nt] = zero16();
  auto gemm2 = [&](int slot, const u32x4 (&hA)[MT][2]) {
    const unsigned base = slot * SLOT;
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int nt = 0; nt < NTN; ++nt) {
        const u32x4 Bv = cat(lds_read_tr(base + offB[s][0][nt]), lds_read_tr(base + offB[s][1][nt]));
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) o[mt][nt] = mfma<BF16>(hA[mt][s], Bv, o[mt][nt]);
      }
  };
  auto activate = [&](const f32x16 (&z)[MT], u32x4 (&hA)[MT][2]) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int w = 0; w < 4; ++w)
          hA[mt][s][w] = pack2<BF16>(act_f<ACT>(z[mt][8 * s + 2 * w]), act_f<ACT>(z[mt][8 * s + 2 * w + 1]));
  };

  // ---- prologue ----
  load_chunk(0);
  store_chunk(0);
  if (NC > 1) {
    load_chunk(1);
    store_chunk(1);
  }
  __syncthreads();
  f32x16 zc[MT];
  gemm1(0, zc);
  u32x4 hp[MT][2];

  // iteration body; G1: compute Z^T(c+1), G2: accumulate h(c-1) W2c(c-1)
  auto iter = [&](auto G1, auto G2, int c) {
    constexpr bool DO_G1 = decltype(G1)::value;
    constexpr bool DO_G2 = decltype(G2)::value;
    load_chunk(c + 2 < NC ? c + 2 : NC - 1);
    f32x16 zn[MT];
    if constexpr (DO_G1) gemm1((c + 1) & 3, zn);
    if constexpr (DO_G2) gemm2((c - 1) & 3, hp);
    activate(zc, hp);
    store_chunk((c + 2) & 3);
    __syncthreads();
    if constexpr (DO_G1) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) zc[mt] = zn[mt];
    }
  };
  if (NC == 1) {
    activate(zc, hp);
  } else {
    iter(std::true_type{}, std::false_type{}, 0);
    for (int c = 1; c < NC - 1; ++c) iter(std::true_type{}, std::true_type{}, c);
    iter(std::false_type{}, std::true_type{}, NC - 1);
  }
  gemm2((NC - 1) & 3, hp);

  // ---- epilogue: O tile (C layout: lane = column d, rows 8(i/4) + 4g + i%4) ----
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int b = b_wave + mt * 32 + 8 * (i >> 2) + 4 * g + (i & 3);
      if (b < B) {
#pragma unroll
        for (int nt = 0; nt < NTN; ++nt) Oh[(size_t)b * D + nt * 32 + l32] = from_f32<BF16>(o[mt][nt][i]);
      }
    }
}

// ------------------------------------------------------------------------------------
// launcher
// ------------------------------------------------------------------------------------
template <bool BF16, int D, int ACT, int NW, int MT>
static hipError_t launch_fwd_t(const FwdArgs& a, hipStream_t st) {
  constexpr int BB = NW * MT * 32;
  const int tiles_per_head = (int)((a.B + BB - 1) / BB);
  const long long grid = (long long)tiles_per_head * a.H;
  if (grid <= 0) return hipSuccess;
  if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
  const size_t lds = 4u * 128u * D;
  auto k = fwd_kernel<BF16, D, ACT, NW, MT>;
  hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(NW * 64), lds, st, (const u16*)a.x, (const u16*)a.w1,
                     (const u16*)a.w2, (u16*)a.o, (int)a.B, (int)a.E, tiles_per_head);
  return hipGetLastError();
}

template <bool BF16, int D, int ACT>
static hipError_t launch_fwd_d(const FwdArgs& a, hipStream_t st) {
  // Tile choice: 4 waves x 64 rows when the grid still covers the chip, else 32 rows.
  const long long big_tiles = ((a.B + 255) / 256) * a.H;
  if (big_tiles >= 2 * 256) return launch_fwd_t<BF16, D, ACT, 4, 2>(a, st);
  return launch_fwd_t<BF16, D, ACT, 4, 1>(a, st);
}

template <bool BF16, int D>
static hipError_t launch_fwd_a(const FwdArgs& a, hipStream_t st) {
  switch (a.act) {
    case ACT_SILU: return launch_fwd_d<BF16, D, ACT_SILU>(a, st);
    case ACT_LEAKY: return launch_fwd_d<BF16, D, ACT_LEAKY>(a, st);
    case ACT_SIGMOID: return launch_fwd_d<BF16, D, ACT_SIGMOID>(a, st);
    default: return launch_fwd_d<BF16, D, ACT_NONE>(a, st);
  }
}

hipError_t launch_fwd(const FwdArgs& a, hipStream_t st) {
  if (a.bf16) {
    if (a.D == 128) return launch_fwd_a<true, 128>(a, st);
    return launch_fwd_a<true, 64>(a, st);
  }
  if (a.D == 128) return launch_fwd_a<false, 128>(a, st);
  return launch_fwd_a<false, 64>(a, st);
}

}  // namespace fmlp
