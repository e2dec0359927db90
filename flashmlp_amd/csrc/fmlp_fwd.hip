// FlashMLP forward kernel for gfx950 (MI355X).
//
// Computes, per head h and B-tile of rows:  O = act(X W1) W2  with fp32 accumulation,
// casting act(Z) to the io dtype before the second contraction (the reference's cast
// point, flashmlp.py:137-150) and O to the io dtype at the store (flashmlp.py:157).
// The (H, B, E) intermediate never leaves registers.
//
// Per workgroup: D/16 waves, each owning one 32-row M-tile (256 rows per workgroup at
// D = 128, 128 at D = 64); two waves per SIMD at D = 128, three at D = 64 (below).
//   * X rows live in registers for the whole kernel, already in the MFMA B-operand layout
//     of Z^T = W1c^T X^T (lane = row b, 8 consecutive d).
//   * E is walked in 32-column chunks. Chunk k's W1c (D x 32) and W2c (32 x D) tiles are
//     staged in an LDS ring of 8 slots; both are read with ds_read_b64_tr_b16, which
//     yields the K-contiguous operands straight from the natural row-major tiles.
//   * Z^T is produced in the MFMA C layout (lane = column b), which is exactly the A
//     operand layout of O += h W2c (lane = row b), so h never round-trips through LDS.
//   * Software pipeline, iteration c:  Z^T(c+1) = W1c(c+1)^T X^T  and  O += h(c-1) W2c(c-1)
//     on the matrix cores while h(c) = act(Z^T(c)) runs on the VALU. Chunk c+5 is loaded
//     straight into its LDS slot (buffer loads with the LDS destination, no registers and
//     no LDS store instructions); one workgroup barrier per two chunks.
#include "fmlp_device.h"
#include "fmlp_launch.h"
#include <algorithm>
#include <type_traits>

namespace fmlp {

// LDS tiles (64-byte rows, no swizzle: every access below is a 4-row x 64-byte block per
// 32-lane phase, which covers all 64 banks once):
//   W1c  [D][32]           row d = W1[h][d][32c .. 32c+31]
//   W2c  [D/32][32][32]    block nt, row e = W2[h][32c + e][32nt .. 32nt+31]
// Waves per workgroup: one 32-row M-tile each, so that the workgroup's threads cover a chunk's
// 4 D pieces of W1c and of W2c exactly once (NT == 4 D); two waves per SIMD either way.
// ES = 2 (E split, D = 64 only, for grids that leave CUs idle): the workgroup holds two such
// sets of waves on the same rows, each walking half of the E-chunks through a ring of its own
// (one workgroup per CU, two waves per SIMD instead of one); the two partial O tiles are added
// through LDS at the end. ES = 4 with NWP = 2 (D = 64, smaller grids still): 64-row tiles, four
// sets of two waves, each walking a quarter of the E-chunks through a 4-slot ring of its own;
// the partial tiles are added in part order.
// Split tiles (fwd_plan): the last n_split tiles in row-block-major order (tile (h, bt) at
// bt H + h; the ragged last tiles of the heads first) are split; the first n_main workgroups
// each own one of the other tiles, enumerated head by head (split_tile / main_tile); every later
// workgroup owns one of xs E-ranges of nct chunks of split tile (b - n_main) / xs and stores its
// fp32 partial O tile to ws (one [BB][D] block per workgroup), which fwd_reduce_kernel sums in
// part order and rounds.
struct TileId {
  int h, bt;
};
// split tile s of n_split (H heads, T tiles per head)
__device__ __forceinline__ TileId split_tile(int s, int n_split, int H, int T) {
  const int t = H * T - n_split + s;
  return TileId{t % H, t / H};
}
// whole tile m: rem = n_split = a H + b leaves heads h < H - b with T - a tiles, the others T - a - 1
__device__ __forceinline__ TileId main_tile(int m, int n_split, int H, int T) {
  const int a = n_split / H, b = n_split - a * H;
  const int first = (H - b) * (T - a);
  if (m < first) return TileId{m / (T - a), m % (T - a)};
  const int m2 = m - first, tb = T - a - 1;
  return TileId{H - b + m2 / tb, m2 % tb};
}
// Waves per workgroup: D / 16 up to D = 128 (two waves per SIMD, the threads covering a chunk's
// 4 D pieces of W1c and of W2c once); 4 at D = 256 (one wave per SIMD, whose O accumulators alone
// take 128 registers; each thread loads 4 pieces per region).
__host__ __device__ constexpr int fwd_waves(int D) { return D <= 128 ? D / 16 : 4; }
// OC: waves per SIMD the kernel is built for. Two up to D = 128 (each workgroup with an 8-slot
// ring); at D = 64 without the E split three, each workgroup then with a 4-slot ring (32 KB) so
// that three fit on a CU: the D = 64 kernel is VALU-issue bound (two activation elements per
// MFMA) and a third wave per SIMD hides more of its latencies (measured on MI355X at H=8
// B=65536 D=64 E=2048, fp16 sigmoid: forward 360 -> 343 us; a 6-slot ring spills registers
// there and four waves per SIMD do not fit in 128 registers without spills); one at D = 256.
__host__ __device__ constexpr int fwd_wpe(int D, int OC) { return D <= 128 ? OC : 1; }
// ring geometry: slots (chunks of 128 D bytes), chunk iterations per workgroup barrier and chunks
// loaded ahead; at D = 256 a chunk is 32 KB, so four slots, a barrier per chunk, two ahead, and
// the same for the 4-slot rings of the higher-occupancy D = 64 builds
constexpr int FWD_PF = 4;  // chunks loaded ahead with one barrier per chunk (D <= 128)
__host__ __device__ constexpr bool fwd_small_ring(int D, int OC, int ES = 1) { return D > 128 || OC > 2 || ES > 2; }
__host__ __device__ constexpr int fwd_nslot(int D, int OC, int ES = 1) { return fwd_small_ring(D, OC, ES) ? 4 : 8; }
__host__ __device__ constexpr int fwd_sb(int D, int OC, int ES = 1) { return fwd_small_ring(D, OC, ES) ? 1 : 2; }
__host__ __device__ constexpr int fwd_pf(int D, int OC, int ES = 1) {
  return fwd_small_ring(D, OC, ES) ? fwd_nslot(D, OC, ES) - 2 : FWD_PF + fwd_sb(D, OC, ES) - 1;
}

template <bool BF16, int D, int ACT, int ES, int OC = 2, int NWP = fwd_waves(D)>
__global__ void __launch_bounds__(NWP * ES * 64) __attribute__((amdgpu_waves_per_eu(fwd_wpe(D, OC), fwd_wpe(D, OC))))
fwd_kernel(const u16* __restrict__ X, const u16* __restrict__ W1, const u16* __restrict__ W2,
           void* __restrict__ O, int B, int E, int H, int tiles_per_head, int outf32, int n_main, int n_split,
           int xs, int nct, float* __restrict__ ws) {
  constexpr int NW = NWP, NT = NW * 64;  // waves, threads of one E part
  constexpr int KS = D / 16;           // K steps of GEMM1 (= GEMM2 operand count 2 * D/32)
  constexpr int NTN = D / 32;          // N tiles of GEMM2
  constexpr int BB = NW * 32;          // rows per workgroup (32 per wave)
  static_assert(ES == 1 || (ES == 2 && D == 64) || (ES == 4 && D == 64 && NWP == 2), "E split");
  static_assert(NWP == fwd_waves(D) || (NWP == 2 && ES == 4), "waves per E part");
  constexpr unsigned SLOT = 128u * D;  // bytes per ring slot: W1c (64*D) + W2c (64*D)
  constexpr unsigned W2OFF = 64u * D;
  // SB: chunk iterations per workgroup barrier. The loads run SB - 1 chunks further ahead so
  // that a barrier covers the SB chunks read after it (measured on MI355X at cfg4: SB = 2 is
  // about 1 % faster than a barrier per chunk).
  static_assert(OC == 2 || (D == 64 && ES == 1 && OC == 3), "occupancy");
  constexpr int SB = fwd_sb(D, OC, ES);
  constexpr int NSLOT = fwd_nslot(D, OC, ES), PF = fwd_pf(D, OC, ES);
  constexpr int NPR = 4 * D / NT;  // 16-byte pieces per thread per region (W1c or W2c) of a chunk
  static_assert(SB == 1 || SB == 2, "barrier spacing");
  static_assert(PF >= 2 && PF <= NSLOT - 2 - (SB - 1) && (NSLOT & (NSLOT - 1)) == 0, "ring");
  auto rslot = [](int c) -> unsigned { return (unsigned)(c & (NSLOT - 1)); };  // ring slot of chunk c

  const int lane = threadIdx.x & 63;
  const int part = ES == 1 ? 0 : __builtin_amdgcn_readfirstlane((int)threadIdx.x / NT);  // E part
  const int tid = threadIdx.x - part * NT;  // thread within the part
  // wave within the part, wave-uniform for the compiler: the chunk loads' LDS addresses and
  // row bases then stay in scalar registers (1.5 % faster forward at cfg4 and cfg5s)
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = lane >> 4, i16 = lane & 15, g = lane >> 5, l32 = lane & 31;
  // this workgroup's tile and E-range [cb, ce) of chunks (all of E for a whole tile)
  const int bid = blockIdx.x;
  const bool split = bid >= n_main;
  int cb = 0, ce = (E + 31) >> 5, u = 0;
  TileId tile;
  if (!split) {
    tile = main_tile(xcd_remap(bid, n_main), n_split, H, tiles_per_head);
  } else {
    u = bid - n_main;
    const int s = u / xs;
    tile = split_tile(s, n_split, H, tiles_per_head);
    cb = (u - s * xs) * nct;
    ce = min(ce, cb + nct);
  }
  const int h = tile.h, bt = tile.bt;
  // chunks of this part: global chunk c0 + c for c = 0 .. NC - 1 (the last part's last chunks
  // may lie past the range: they load as zeros and add nothing)
  const int NC = (ce - cb + ES - 1) / ES;
  const int c0 = cb + part * NC;
  const int e_end = min(E, ce * 32);  // columns of W1 (rows of W2) this workgroup reads
  const unsigned RB = (unsigned)part * NSLOT * 128u * D;  // this part's ring

  const u16* Xh = X + (size_t)h * B * D;
  const u16* W1h = W1 + (size_t)h * D * E;
  const u16* W2h = W2 + (size_t)h * E * D;
  const int b_wave = bt * BB + wave * 32;

  // ---- chunk staging: buffer-to-LDS loads, PF chunks ahead into an NSLOT-slot ring ----
  // NPR 16-byte pieces per thread per region: piece p = tid + k NT of W1c lands at slot offset
  // 16 p (row d = p / 4, columns 8 (p % 4) ..), piece p of W2c at W2OFF + 16 p (block p / 128,
  // row (p / 4) % 32, columns 32 (p / 128) + 8 (p % 4) ..). Columns past E (and every piece of a
  // chunk past the last) are out of range and land as zeros.
  static_assert(NPR * NT == 4 * D, "the threads cover a region's pieces");
  int colq[NPR];
  unsigned dOffW1[NPR], dOffW2[NPR];
#pragma unroll
  for (int k = 0; k < NPR; ++k) {
    const unsigned p = (unsigned)(tid + k * NT);
    colq[k] = (int)(p & 3u) * 8;
    dOffW1[k] = (p >> 2) * (unsigned)E * 2u + (p & 3u) * 16u;
    dOffW2[k] = ((p >> 2) & 31u) * (D * 2u) + (p >> 7) * 64u + (p & 3u) * 16u;
  }
  auto dma_chunk = [&](int c) {
    const int cg = c0 + c;
    const int lim = e_end - cg * 32;
    const int rem = D * E * 2 - 64 * cg;
    const i32x4 r1 = make_rsrc_words(W1h + (size_t)cg * 32, rem > 0 ? rem : 0);
    const i32x4 r2 = make_rsrc_words(W2h + (size_t)cg * 32 * D, clamp0(lim, 32) * D * 2);
    const int slot = (int)RB + (int)rslot(c) * (int)SLOT + wave * 1024;
#pragma unroll
    for (int k = 0; k < NPR; ++k) {
      buf_load16_lds(r1, colq[k] < lim ? dOffW1[k] : BUF_OOB, slot + k * NT * 16);
      buf_load16_lds(r2, dOffW2[k], slot + (int)W2OFF + k * NT * 16);
    }
  };
  // end of a chunk: the LDS stores are retired and visible after the barrier; the loads of
  // the chunk after next stay in flight (their data is waited for where it is stored)
  auto chunk_end = [&]() {
    wait_vmcnt<2 * NPR * (PF - 1 - SB)>();  // this wave's pieces of the SB chunks read next
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

  // ---- prologue: chunks 0 .. PF-1 requested, chunk 0 waited for, Z^T(0) ----
#pragma unroll
  for (int c = 0; c < PF; ++c) dma_chunk(c);
  wait_vmcnt<2 * NPR * (PF - 2)>();  // chunks 0 and 1
  __builtin_amdgcn_s_waitcnt(0xC07F);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
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
  for (int ks = 0; ks < KS; ++ks) sa.z = mfma<BF16>(opndA(RB, ks), xr[ks], sa.z);

  // Iteration c (G1: Z^T(c+1) = W1c(c+1)^T X^T, G2: O += h(c-1) W2c(c-1), act: h(c)), reading
  // `in` (Z^T(c), h(c-1)) and writing `out` (Z^T(c+1), h(c)). Written as a fixed sequence of
  // steps: each step issues one MFMA, the operand reads of the MFMA two steps later and a
  // share of the activation; sched_barrier keeps the order.
  auto iter = [&](auto G1, auto G2, auto SYNC, int c, St& in, St& out) {
    constexpr bool DO_G1 = decltype(G1)::value;
    constexpr bool DO_G2 = decltype(G2)::value;
    constexpr int N1 = DO_G1 ? KS : 0, N2 = DO_G2 ? KS : 0, NOPS = N1 + N2;
    // activation elements of step j: [16 j / NOPS, 16 (j + 1) / NOPS) (one or two per step at
    // D <= 128, one every other step at D = 256)
    const unsigned base1 = RB + rslot(c + 1) * SLOT, base2 = RB + rslot(c - 1) * SLOT;

    // chunk c+PF is requested straight into its LDS slot (PF chunks ahead of the one read)
    dma_chunk(c + PF);

    // op j: G1 and G2 alternate when both are present
    auto is_g1 = [&](int j) { return DO_G1 && (!DO_G2 || (j % 2 == 0)); };
    auto idx = [&](int j) { return (DO_G1 && DO_G2) ? j / 2 : j; };
    auto fetch = [&](int j) {
      const int k = idx(j);
      return is_g1(j) ? opndA(base1, k) : opndB(base2, k / NTN, k % NTN);
    };
    constexpr int PDX = NOPS < 2 ? NOPS : 2;  // operand reads two steps ahead
    u32x4 ring[PDX + 1];
#pragma unroll
    for (int j = 0; j < PDX; ++j) ring[j] = fetch(j);
    float hv[16];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < NOPS; ++j) {
      const u32x4 cur = ring[j % (PDX + 1)];
      if (j + PDX < NOPS) ring[(j + PDX) % (PDX + 1)] = fetch(j + PDX);
      const int k = idx(j);
      if (is_g1(j)) {  // k == 0 starts the chain from a literal zero accumulator
        out.z = mfma<BF16>(cur, xr[k], k == 0 ? zero16() : out.z);
      } else {
        const int s = k / NTN, nt = k % NTN;
        o[nt] = mfma<BF16>(s == 0 ? in.h0 : in.h1, cur, o[nt]);
      }
#pragma unroll
      for (int e = 16 * j / NOPS; e < 16 * (j + 1) / NOPS; ++e) {
        hv[e] = act_f<ACT>(in.z[e]);
        if (e & 1) {
          const unsigned pk = pack2<BF16>(hv[e - 1], hv[e]);
          const int w = (e >> 1) & 3;
          if (e < 8) out.h0[w] = pk; else out.h1[w] = pk;
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (decltype(SYNC)::value) chunk_end();
  };
  auto last_gemm2 = [&](const St& st) {
    const unsigned base2 = RB + rslot(NC - 1) * SLOT;
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
    // barriers after iteration 0 and after every second iteration from there (SB = 2), or
    // after every iteration (SB = 1); the tail iterations read only chunks the last barrier
    // covered, so with SB = 2 they need none
    const std::integral_constant<bool, SB == 1> S1{};
    iter(T, F, T, 0, sa, sb);
    int c = 1;
    for (; c + 2 < NC; c += 2) {
      iter(T, T, S1, c, sb, sa);
      iter(T, T, T, c + 1, sa, sb);
    }
    if (c + 2 == NC) {  // one more full iteration, then the last
      iter(T, T, S1, c, sb, sa);
      iter(F, T, S1, c + 1, sa, sb);
      last_gemm2(sb);
    } else {            // c == NC - 1
      iter(F, T, S1, c, sb, sa);
      last_gemm2(sa);
    }
  }

  wait_vmcnt<0>();  // chunks past the last are still landing (as zeros)
  if constexpr (ES > 1) {  // parts 1 .. ES-1 hand their partial O tiles to part 0 through LDS (the rings)
    asm volatile("" ::: "memory");
    __syncthreads();
    // per wave NTN x 4 x [64 lanes][16 bytes], one region per handing part
    const int ob = wave * (NTN * 4096) + (part > 0 ? part - 1 : 0) * (NW * NTN * 4096);
    static_assert((ES - 1) * NW * NTN * 4096 <= ES * NSLOT * (int)SLOT, "the partial tiles fit the rings");
    if (part > 0) {
#pragma unroll
      for (int nt = 0; nt < NTN; ++nt)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4)
          lds_write16(ob + ((nt * 4 + i4) * 64 + lane) * 16,
                      u32x4{__float_as_uint(o[nt][4 * i4]), __float_as_uint(o[nt][4 * i4 + 1]),
                            __float_as_uint(o[nt][4 * i4 + 2]), __float_as_uint(o[nt][4 * i4 + 3])});
    }
    __syncthreads();
    if (part > 0) return;
#pragma unroll
    for (int p = 1; p < ES; ++p)  // in part order
#pragma unroll
      for (int nt = 0; nt < NTN; ++nt)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
          const u32x4 v = lds_read16(ob + (p - 1) * (NW * NTN * 4096) + ((nt * 4 + i4) * 64 + lane) * 16);
#pragma unroll
          for (int j = 0; j < 4; ++j) o[nt][4 * i4 + j] += __uint_as_float(v[j]);
        }
  }
  // ---- epilogue: O tile (C layout: lane = column d, rows 8(i/4) + 4g + i%4); fp32 sums
  // when the caller asked for them (FMLP_OUT_F32), else rounded to the io dtype; a split
  // tile's partial as fp32 rows of its workspace block ----
  if (split)
    store_rows<BF16, D>(o, ws, (size_t)u * BB * D, B - bt * BB, wave * 32, g, l32, 1);
  else
    store_rows<BF16, D>(o, O, (size_t)h * B * D, B, b_wave, g, l32, outf32);
}

// Sum of the split tiles' partials: O rows of split tile s = sum over p < xs of
// ws[s xs + p] (in p order), fp32 when outf32, else rounded to the io dtype. Four columns per
// thread; all xs (<= FWD_XS_MAX) partials are loaded before the sum, so their latencies overlap.
constexpr int FWD_XS_MAX = 16;
template <bool BF16>
__global__ void __launch_bounds__(64)
fwd_reduce_kernel(const float* __restrict__ ws, void* __restrict__ O, int B, int D, int BB, int H, int tiles_per_head,
                  int xs, int n_split, int outf32) {
  const int DQ = D >> 2;
  const long long items = (long long)n_split * BB * DQ;
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long it = (long long)blockIdx.x * blockDim.x + threadIdx.x; it < items; it += stride) {
    const int q = (int)(it % DQ);
    const long long sr = it / DQ;
    const int r = (int)(sr % BB), s = (int)(sr / BB);
    const TileId tile = split_tile(s, n_split, H, tiles_per_head);
    const int h = tile.h, b = tile.bt * BB + r;
    if (b >= B) continue;
    const float* src = ws + ((size_t)s * xs * BB + r) * D + 4 * q;
    float4 v[FWD_XS_MAX];
#pragma unroll
    for (int p = 0; p < FWD_XS_MAX; ++p)
      if (p < xs) v[p] = *(const float4*)(src + (size_t)p * BB * D);
    float4 acc = v[0];
#pragma unroll
    for (int p = 1; p < FWD_XS_MAX; ++p) {
      if (p < xs) {
        acc.x += v[p].x;
        acc.y += v[p].y;
        acc.z += v[p].z;
        acc.w += v[p].w;
      }
    }
    const size_t i = ((size_t)h * B + b) * D + 4 * q;
    if (outf32) {
      *(float4*)((float*)O + i) = acc;
    } else {
      const u32x2 v = {pack2<BF16>(acc.x, acc.y), pack2<BF16>(acc.z, acc.w)};
      *(u32x2*)((u16*)O + i) = v;
    }
  }
}

// ------------------------------------------------------------------------------------
// launcher
// ------------------------------------------------------------------------------------
// Work split of a forward call on num_cus CUs. Tiles of BB rows (256 at D = 128, 128 at
// D = 64), R = H ceil(B / BB) of them (at most 2^31 - 1, so every tile index fits an int). One tile per workgroup, one workgroup per CU at a time
// (D = 128, or D = 64 with the in-workgroup E split) or two (D = 64 without it). A last round
// of at most N / 4 tiles after full ones (e.g. one ragged tile per head just past a multiple
// of the CU count) costs nearly as much as a full round, so those tiles are split over E
// across workgroups, in up to min(N / rem, 16) parts of at least 4 chunks each (two per wave
// set with the in-workgroup split); the parts' fp32 partials go to the caller's workspace and
// a second launch sums them. At D = 64 the full round then runs with the in-workgroup split
// (one tile per CU). Measured on MI355X at H=8 B=4097 D=64 E=2048: 43.9 us unsplit, 33.0 us
// for the split launch. Small grids (fewer tiles than CUs) gain nothing from it: their tiles'
// time is mostly fixed latency (12.5 vs 11.4 us at H=12 B=1024 D=64 E=768, before the sum).
// FMLP_FWD_XS=0 (read once per process) turns the cross-workgroup split off.
FwdPlan fwd_plan(int64_t H, int64_t B, int64_t D, int64_t E, int num_cus, size_t max_ws) {
  FwdPlan p{};
  const long long BB = 32 * fwd_waves((int)D), T = (B + BB - 1) / BB, R = H * T, N = num_cus > 0 ? num_cus : 1;
  const long long nch = (E + 31) / 32;
  // in-workgroup split at D = 64 when the tiles fit on the CUs at one workgroup each (the
  // unsplit kernel would leave a SIMD with one wave) and each part gets at least two chunks;
  // FMLP_FWD_SPLIT (read once per process): 0 = never, 1 = whenever E allows, else this rule
  static const int force = env_int("FMLP_FWD_SPLIT", -1);
  static const int xs_env = env_int("FMLP_FWD_XS", -1);
  p.es = (D == 64 && E > 64 && (force == 1 || (force != 0 && R <= N))) ? 2 : 1;
  p.n_main = R;
  p.xs = 1;
  p.nct = (int)nch;
  // 64-row tiles in four E parts of two waves: twice the workgroups of the split above, each
  // walking a quarter of the chunks, when they still fit on the CUs at one each and every part
  // gets at least two chunks. These grids are latency-bound (one round, short chunk loops):
  // measured on MI355X at H=12 B=1024 D=64 E=768 fp16, forward 11.6 -> 8.8 us, at H=8 B=512
  // E=512 bf16 8.8 -> 6.9 us. FMLP_FWD_T64=0 (read once per process) keeps 128-row tiles.
  static const int t64_env = env_int("FMLP_FWD_T64", 1);
  const long long R64 = H * ((B + 63) / 64);
  if (t64_env != 0 && p.es == 2 && force != 1 && R <= N && R64 <= N && nch >= 8) {
    p.es = 4;
    p.nwp = 2;
    p.n_main = R64;
    return p;
  }
  if (xs_env == 0 || R <= 0) return p;
  long long cand = 0;
  int es = p.es;
  if (R > N) {
    if (D == 64) {
      if (R - N <= N / 4 && E > 64 && force != 0) {
        cand = R - N;
        es = 2;
      }
    } else if (R % N != 0 && R % N <= N / 4) {
      cand = R % N;
    }
  }
  if (cand <= 0) return p;
  long long xs = std::min<long long>(std::min<long long>(N / cand, nch / 4), FWD_XS_MAX);
  if (xs < 2) return p;
  const long long nct = (nch + xs - 1) / xs;
  xs = (nch + nct - 1) / nct;
  const size_t ws = (size_t)cand * (size_t)xs * (size_t)BB * (size_t)D * sizeof(float);
  if (ws > max_ws || R - cand + cand * xs > 0x7fffffffLL) return p;
  p.es = es;
  p.n_main = R - cand;
  p.n_split = (int)cand;
  p.xs = (int)xs;
  p.nct = (int)nct;
  p.ws_bytes = ws;
  return p;
}

template <bool BF16, int D, int ACT, int ES, int OC = 2, int NWP = fwd_waves(D)>
static hipError_t launch_fwd_e(const FwdArgs& a, const FwdPlan& p, int tiles_per_head, hipStream_t st) {
  const size_t lds = (size_t)ES * fwd_nslot(D, OC, ES) * 128u * D;
  auto k = fwd_kernel<BF16, D, ACT, ES, OC, NWP>;
  static std::atomic<unsigned long long> lds_set{0};
  hipError_t e = set_lds_once((const void*)k, (int)lds, lds_set);
  if (e != hipSuccess) return e;
  const long long grid = p.n_main + (long long)p.n_split * p.xs;
  hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(64 * ES * NWP), lds, st, (const u16*)a.x,
                     (const u16*)a.w1, (const u16*)a.w2, a.o, (int)a.B, (int)a.E, (int)a.H, tiles_per_head,
                     a.out_f32 ? 1 : 0, (int)p.n_main, p.n_split, p.xs, p.nct, (float*)a.ws);
  if ((e = hipGetLastError()) != hipSuccess || p.n_split == 0) return e;
  return launch_tile_reduce((const float*)a.ws, a.o, BF16, (int)a.B, D, 32 * NWP, (int)a.H, tiles_per_head,
                            p.xs, p.n_split, a.out_f32 ? 1 : 0, st);
}

hipError_t launch_tile_reduce(const float* ws, void* out, bool bf16, int B, int D, int BB, int H, int T, int xs,
                              int n_split, int outf32, hipStream_t st) {
  if (xs < 1 || xs > FWD_XS_MAX || D % 4 != 0) return hipErrorInvalidValue;
  const long long items = (long long)n_split * BB * (D / 4);
  const long long blocks = std::min<long long>((items + 63) / 64, 8192);
  if (blocks <= 0) return hipSuccess;
  if (bf16)
    hipLaunchKernelGGL(fwd_reduce_kernel<true>, dim3((unsigned)blocks), dim3(64), 0, st, ws, out, B, D, BB, H, T, xs,
                       n_split, outf32);
  else
    hipLaunchKernelGGL(fwd_reduce_kernel<false>, dim3((unsigned)blocks), dim3(64), 0, st, ws, out, B, D, BB, H, T,
                       xs, n_split, outf32);
  return hipGetLastError();
}

template <bool BF16, int D, int ACT>
static hipError_t launch_fwd_t(const FwdArgs& a, hipStream_t st) {
  constexpr int BB0 = 32 * fwd_waves(D);
  if ((a.B + BB0 - 1) / BB0 * a.H <= 0) return hipSuccess;
  if ((a.B + 63) / 64 * a.H > 0x7fffffffLL) return hipErrorInvalidValue;
  const FwdPlan p = fwd_plan(a.H, a.B, D, a.E, a.num_cus, a.ws != nullptr ? a.ws_bytes : 0);
  const int BB = 32 * (p.nwp > 0 ? p.nwp : fwd_waves(D));
  const int tiles_per_head = (int)((a.B + BB - 1) / BB);
  if constexpr (D == 64) {
    if (p.es == 4) return launch_fwd_e<BF16, D, ACT, 4, 2, 2>(a, p, tiles_per_head, st);
    if (p.es == 2) return launch_fwd_e<BF16, D, ACT, 2>(a, p, tiles_per_head, st);
    // FMLP_FWD_OCC=2 (read once per process) keeps two waves per SIMD
    static const int occ = env_int("FMLP_FWD_OCC", 3);
    if (occ != 2) return launch_fwd_e<BF16, D, ACT, 1, 3>(a, p, tiles_per_head, st);
  }
  return launch_fwd_e<BF16, D, ACT, 1>(a, p, tiles_per_head, st);
}

template <bool BF16, int D>
static hipError_t launch_fwd_a(const FwdArgs& a, hipStream_t st) {
  switch (a.act) {
    case ACT_SILU: return launch_fwd_t<BF16, D, ACT_SILU>(a, st);
    case ACT_LEAKY: return launch_fwd_t<BF16, D, ACT_LEAKY>(a, st);
    case ACT_SIGMOID: return launch_fwd_t<BF16, D, ACT_SIGMOID>(a, st);
    default: return launch_fwd_t<BF16, D, ACT_NONE>(a, st);
  }
}

hipError_t launch_fwd(const FwdArgs& a, hipStream_t st) {
  if (a.bf16) {
    if (a.D == 256) return launch_fwd_a<true, 256>(a, st);
    if (a.D == 128) return launch_fwd_a<true, 128>(a, st);
    return launch_fwd_a<true, 64>(a, st);
  }
  if (a.D == 256) return launch_fwd_a<false, 256>(a, st);
  if (a.D == 128) return launch_fwd_a<false, 128>(a, st);
  return launch_fwd_a<false, 64>(a, st);
}

}  // namespace fmlp
