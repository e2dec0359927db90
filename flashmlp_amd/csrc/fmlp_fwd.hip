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

// LDS tiles (64-byte rows, no swizzle: every access below is a 4-row x 64-byte block per
// 32-lane phase, which covers all 64 banks once):
//   W1c  [D][32]           row d = W1[h][d][32c .. 32c+31]
//   W2c  [D/32][32][32]    block nt, row e = W2[h][32c + e][32nt .. 32nt+31]
template <bool BF16, int D, int ACT>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
fwd_kernel(const u16* __restrict__ X, const u16* __restrict__ W1, const u16* __restrict__ W2,
           void* __restrict__ O, int B, int E, int tiles_per_head, int outf32) {
  constexpr int NW = 4, NT = NW * 64;  // waves, threads
  constexpr int KS = D / 16;           // K steps of GEMM1 (= GEMM2 operand count 2 * D/32)
  constexpr int NTN = D / 32;          // N tiles of GEMM2
  constexpr int BB = NW * 32;          // rows per workgroup (32 per wave)
  constexpr unsigned SLOT = 128u * D;  // bytes per ring slot: W1c (64*D) + W2c (64*D)
  constexpr unsigned W2OFF = 64u * D;
  constexpr int PPT = 8 * D / NT;      // 16-byte pieces per thread per chunk (half W1c, half W2c)
  static_assert(PPT % 2 == 0, "pieces per thread");

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int G = lane >> 4, i16 = lane & 15, g = lane >> 5, l32 = lane & 31;
  const int t = xcd_remap(blockIdx.x, gridDim.x);
  const int h = t / tiles_per_head, bt = t - h * tiles_per_head;
  const int NC = (E + 31) >> 5;

  const u16* Xh = X + (size_t)h * B * D;
  const u16* W1h = W1 + (size_t)h * D * E;
  const u16* W2h = W2 + (size_t)h * E * D;
  const int b_wave = bt * BB + wave * 32;

  // ---- chunk staging: global -> registers (one chunk ahead) -> LDS ----
  // Branch-free buffer loads: W2c rows past E fall outside the chunk's resource; W1c
  // columns past E (last chunk when E % 32 != 0) get an out-of-range offset. Chunks past
  // the last one are loaded but never used.
  u32x4 stg[PPT];
  const unsigned colq = (tid & 3) * 8;  // first column of this thread's W1c pieces
  unsigned offW1g[PPT / 2], offW2g[PPT / 2];
#pragma unroll
  for (int k = 0; k < PPT / 2; ++k) {
    const unsigned p = tid + k * NT;
    offW1g[k] = (p >> 2) * (unsigned)E * 2u + (p & 3u) * 16u;                   // row d, piece q
    offW2g[k] = ((p >> 2) & 31u) * (D * 2u) + (p >> 7) * 64u + (p & 3u) * 16u;   // row er, block nt, piece q
  }
  struct ChunkSrc {
    Rsrc r1, r2;
    int lim;
  };
  auto chunk_src = [&](int c) {
    ChunkSrc cs;
    cs.lim = E - c * 32;
    cs.r1 = make_rsrc(W1h + (size_t)c * 32, D * E * 2 - 64 * c);
    cs.r2 = make_rsrc(W2h + (size_t)c * 32 * D, clamp0(cs.lim, 32) * D * 2);
    return cs;
  };
  auto load_piece = [&](const ChunkSrc& cs, int k) {
    if (k < PPT / 2) stg[k] = buf_load16(cs.r1, (int)colq < cs.lim ? offW1g[k] : BUF_OOB);
    else stg[k] = buf_load16(cs.r2, offW2g[k - PPT / 2]);
  };
  auto store_piece = [&](int slot, int k) {
    const unsigned base = slot * SLOT;
    const unsigned p = tid + (k % (PPT / 2)) * NT;
    if (k < PPT / 2) lds_write16(base + p * 16u, stg[k]);  // d*64 + q*16
    else lds_write16(base + W2OFF + (p >> 7) * 2048u + ((p >> 2) & 31u) * 64u + (p & 3u) * 16u, stg[k]);
  };
  auto load_chunk = [&](int c) {
    const ChunkSrc cs = chunk_src(c);
#pragma unroll
    for (int k = 0; k < PPT; ++k) load_piece(cs, k);
  };
  auto store_chunk = [&](int slot) {
#pragma unroll
    for (int k = 0; k < PPT; ++k) store_piece(slot, k);
  };
  // end of a chunk: the LDS stores are retired and visible after the barrier; the loads of
  // the chunk after next stay in flight (their data is waited for where it is stored)
  auto chunk_end = [&]() {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  // ---- X rows -> registers (B operand of Z^T = W1c^T X^T: lane = row b, 8 consecutive d) ----
  u32x4 xr[KS];
  {
    const int b = b_wave + l32;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (b < B) v = *(const u32x4*)(Xh + (size_t)b * D + ks * 16 + g * 8);
      xr[ks] = v;
    }
  }

  // lane part of the transposed-read addresses (16-lane group G reads a 4x16 block; lane i16
  // reads row i16/4, columns 4*(i16%4)..+3)
  //   GEMM1 A (W1c^T): rows 16ks + 8g + 4r + i16/4, columns 16(G%2) + 4(i16%4)
  //   GEMM2 B (W2c):   block nt, rows 16s + 8r + 4g + i16/4, columns 16(G%2) + 4(i16%4)
  const unsigned laneA = (8 * g + (i16 >> 2)) * 64 + 32 * (G & 1) + 8 * (i16 & 3);
  const unsigned laneB = W2OFF + (4 * g + (i16 >> 2)) * 64 + 32 * (G & 1) + 8 * (i16 & 3);
  auto opndA = [&](unsigned base, int ks) {
    return cat(lds_read_tr(base + laneA + ks * 1024u), lds_read_tr(base + laneA + ks * 1024u + 256u));
  };
  auto opndB = [&](unsigned base, int s, int nt) {
    const unsigned a = base + laneB + nt * 2048u + s * 1024u;
    return cat(lds_read_tr(a), lds_read_tr(a + 512u));
  };

  f32x16 o[NTN];
#pragma unroll
  for (int nt = 0; nt < NTN; ++nt) o[nt] = zero16();

  // ---- prologue: chunks 0 and 1 in LDS, chunk 2 in registers, Z^T(0) ----
  load_chunk(0);
  store_chunk(0);
  if (NC > 1) {
    load_chunk(1);
    store_chunk(1);
  }
  load_chunk(2);
  chunk_end();
  // Pipeline state carried between iterations: Z^T of the chunk to activate and h of the
  // previous chunk (A operand of O += h W2c, two K steps). Iterations run in pairs with the
  // two state copies swapping roles, so nothing is copied between iterations.
  struct St {
    f32x16 z;
    u32x4 h0, h1;
  };
  St sa, sb;
  sa.z = zero16();
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) sa.z = mfma<BF16>(opndA(0, ks), xr[ks], sa.z);

  // Iteration c (G1: Z^T(c+1) = W1c(c+1)^T X^T, G2: O += h(c-1) W2c(c-1), act: h(c)), reading
  // `in` (Z^T(c), h(c-1)) and writing `out` (Z^T(c+1), h(c)). Written as a fixed sequence of
  // steps: each step issues one MFMA, the operand reads of the MFMA two steps later and a
  // share of the activation; sched_barrier keeps the order.
  auto iter = [&](auto G1, auto G2, int c, St& in, St& out) {
    constexpr bool DO_G1 = decltype(G1)::value;
    constexpr bool DO_G2 = decltype(G2)::value;
    constexpr int N1 = DO_G1 ? KS : 0, N2 = DO_G2 ? KS : 0, NOPS = N1 + N2;
    constexpr int PER = 16 / NOPS;  // activation elements per step
    const unsigned base1 = ((c + 1) & 3) * SLOT, base2 = ((c - 1) & 3) * SLOT;

    // chunk c+2 (loaded during iteration c-1) goes to its slot and chunk c+3 is loaded into
    // the same registers, one 16-byte piece per step (store of piece k at step 2k, its next
    // load at step 2k+1)
    const int sslot = (c + 2) & 3;
    const ChunkSrc cs = chunk_src(c + 3);
    static_assert(2 * PPT <= KS, "staging steps");

    // op j: G1 and G2 alternate when both are present
    auto is_g1 = [&](int j) { return DO_G1 && (!DO_G2 || (j % 2 == 0)); };
    auto idx = [&](int j) { return (DO_G1 && DO_G2) ? j / 2 : j; };
    auto fetch = [&](int j) {
      const int k = idx(j);
      return is_g1(j) ? opndA(base1, k) : opndB(base2, k / NTN, k % NTN);
    };
    u32x4 op0 = fetch(0), op1 = NOPS > 1 ? fetch(1) : op0, op2 = op0;
    float hv[16];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < NOPS; ++j) {
      const u32x4 cur = (j % 3 == 0) ? op0 : (j % 3 == 1) ? op1 : op2;
      if (j + 2 < NOPS) {
        const u32x4 nx = fetch(j + 2);
        if ((j + 2) % 3 == 0) op0 = nx; else if ((j + 2) % 3 == 1) op1 = nx; else op2 = nx;
      }
      if (j < 2 * PPT) {
        if ((j & 1) == 0) store_piece(sslot, j >> 1);
        else load_piece(cs, j >> 1);
      }
      const int k = idx(j);
      if (is_g1(j)) {  // k == 0 starts the chain from a literal zero accumulator
        out.z = mfma<BF16>(cur, xr[k], k == 0 ? zero16() : out.z);
      } else {
        const int s = k / NTN, nt = k % NTN;
        o[nt] = mfma<BF16>(s == 0 ? in.h0 : in.h1, cur, o[nt]);
      }
#pragma unroll
      for (int q = 0; q < PER; ++q) {
        const int e = j * PER + q;
        hv[e] = act_f<ACT>(in.z[e]);
        if (e & 1) {
          const unsigned pk = pack2<BF16>(hv[e - 1], hv[e]);
          const int w = (e >> 1) & 3;
          if (e < 8) out.h0[w] = pk; else out.h1[w] = pk;
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    chunk_end();
  };
  auto last_gemm2 = [&](const St& st) {
    const unsigned base2 = ((NC - 1) & 3) * SLOT;
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int nt = 0; nt < NTN; ++nt) o[nt] = mfma<BF16>(s == 0 ? st.h0 : st.h1, opndB(base2, s, nt), o[nt]);
  };
  if (NC == 1) {
#pragma unroll
    for (int e = 0; e < 16; e += 2) {
      const unsigned pk = pack2<BF16>(act_f<ACT>(sa.z[e]), act_f<ACT>(sa.z[e + 1]));
      if (e < 8) sb.h0[e >> 1] = pk; else sb.h1[(e - 8) >> 1] = pk;
    }
    last_gemm2(sb);
  } else {
    const std::true_type T{};
    const std::false_type F{};
    iter(T, F, 0, sa, sb);
    int c = 1;
    for (; c + 2 < NC; c += 2) {
      iter(T, T, c, sb, sa);
      iter(T, T, c + 1, sa, sb);
    }
    if (c + 2 == NC) {  // one more full iteration, then the last
      iter(T, T, c, sb, sa);
      iter(F, T, c + 1, sa, sb);
      last_gemm2(sb);
    } else {            // c == NC - 1
      iter(F, T, c, sb, sa);
      last_gemm2(sa);
    }
  }

  // ---- epilogue: O tile (C layout: lane = column d, rows 8(i/4) + 4g + i%4); fp32 sums
  // when the caller asked for them (FMLP_OUT_F32), else rounded to the io dtype ----
  if (outf32) {
    float* Oh = (float*)O + (size_t)h * B * D;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int b = b_wave + 8 * (i >> 2) + 4 * g + (i & 3);
      if (b < B) {
#pragma unroll
        for (int nt = 0; nt < NTN; ++nt) Oh[(size_t)b * D + nt * 32 + l32] = o[nt][i];
      }
    }
  } else {
    u16* Oh = (u16*)O + (size_t)h * B * D;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int b = b_wave + 8 * (i >> 2) + 4 * g + (i & 3);
      if (b < B) {
#pragma unroll
        for (int nt = 0; nt < NTN; ++nt) Oh[(size_t)b * D + nt * 32 + l32] = from_f32<BF16>(o[nt][i]);
      }
    }
  }
}

// ------------------------------------------------------------------------------------
// launcher
// ------------------------------------------------------------------------------------
template <bool BF16, int D, int ACT>
static hipError_t launch_fwd_t(const FwdArgs& a, hipStream_t st) {
  constexpr int BB = 128;
  const int tiles_per_head = (int)((a.B + BB - 1) / BB);
  const long long grid = (long long)tiles_per_head * a.H;
  if (grid <= 0) return hipSuccess;
  if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
  const size_t lds = 4u * 128u * D;
  auto k = fwd_kernel<BF16, D, ACT>;
  hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(256), lds, st, (const u16*)a.x, (const u16*)a.w1,
                     (const u16*)a.w2, a.o, (int)a.B, (int)a.E, tiles_per_head, a.out_f32 ? 1 : 0);
  return hipGetLastError();
}

template <bool BF16, int D, int ACT>
static hipError_t launch_fwd_d(const FwdArgs& a, hipStream_t st) {
  // 4 waves x 32 rows per workgroup; two workgroups share a CU (two waves per SIMD)
  return launch_fwd_t<BF16, D, ACT>(a, st);
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
