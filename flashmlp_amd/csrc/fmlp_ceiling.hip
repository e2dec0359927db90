// Sustained bf16 MFMA ceiling of the device (measurement only, not part of the FlashMLP
// path): every wave issues independent v_mfma_f32_32x32x16_bf16 chains with its operands
// held in registers, two waves per SIMD, no memory traffic inside the loop. The rate it
// reaches with random operand bits (versus all-zero operands) is the executed-MFMA rate the
// part sustains at its power limit, the reference point for the kernels' MFMA busy figures.
// Built into its own library (libfmlp_ceiling.so) and used by bench.py --workload mfma_ceiling.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kChains = 4;    // independent accumulators per wave
constexpr int kThreads = 256;  // four waves per workgroup

__device__ __forceinline__ unsigned mix(unsigned x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

// bf16 with a random sign and mantissa and an exponent near 1 (finite for any chain length)
__device__ __forceinline__ __bf16 rnd_bf16(unsigned h) {
  const unsigned short bits = (unsigned short)((h & 0x807fu) | (0x3f00u + ((h >> 8) & 0x80u)));
  return __builtin_bit_cast(__bf16, bits);
}

__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
mfma_ceiling_kernel(float* __restrict__ out, int iters, int zero_data) {
  const unsigned gid = blockIdx.x * kThreads + threadIdx.x;
  bf16x8 a[kChains], b[kChains];
#pragma unroll
  for (int c = 0; c < kChains; ++c)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const unsigned h = mix(gid * 64u + c * 8u + j);
      a[c][j] = zero_data ? (__bf16)0.f : rnd_bf16(h);
      b[c][j] = zero_data ? (__bf16)0.f : rnd_bf16(mix(h));
    }
  f32x16 acc[kChains];
#pragma unroll
  for (int c = 0; c < kChains; ++c)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[c][i] = 0.f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int c = 0; c < kChains; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[c], b[c], acc[c], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < kChains; ++c)
#pragma unroll
    for (int i = 0; i < 16; ++i) s += acc[c][i];
  out[gid] = s;
}

// Sustained MFMA rate with a kernel's other per-MFMA work added: NL 16-byte-per-lane LDS reads
// feeding the A operand (1 KB per wave and read, conflict-free, from a 32 KB LDS tile of random
// bf16) and NV activation-like VALU chains (v_mul, v_exp, v_add, v_rcp, as one sigmoid element)
// per MFMA. 16 MFMAs per iteration, four accumulators, two waves per SIMD. The rate relative to
// the plain loop prices LDS traffic and activation math in MFMA time on a power-limited part.
template <int NL, int NV>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
mfma_mix_kernel(float* __restrict__ out, int iters) {
  __shared__ bf16x8 tile[2048];
  const unsigned gid = blockIdx.x * kThreads + threadIdx.x;
  const int lane = threadIdx.x & 63;
  for (int i = threadIdx.x; i < 2048; i += kThreads)
#pragma unroll
    for (int j = 0; j < 8; ++j) tile[i][j] = rnd_bf16(mix(blockIdx.x * 16384u + i * 8u + j));
  __syncthreads();
  bf16x8 a[16], b[16];
#pragma unroll
  for (int c = 0; c < 16; ++c)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const unsigned h = mix(gid * 256u + c * 8u + j);
      a[c][j] = rnd_bf16(h);
      b[c][j] = rnd_bf16(mix(h));
    }
  float v[2] = {0.01f * lane, 0.5f};
  f32x16 acc[kChains];
#pragma unroll
  for (int c = 0; c < kChains; ++c)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[c][i] = 0.f;
  for (int it = 0; it < iters; ++it) {
    const int base = lane ^ ((it & 1) << 5);  // loop-variant, so the reads stay in the loop
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      bf16x8 A = a[s];
      if constexpr (NL >= 1) A = tile[base + s * 64];
      acc[s % kChains] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, b[s], acc[s % kChains], 0, 0, 0);
#pragma unroll
      for (int q = 0; q < NV; ++q)
        v[q] = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(v[q] * -1.4426950408889634f));
    }
  }
  float t = v[0] + v[1];
#pragma unroll
  for (int c = 0; c < kChains; ++c)
#pragma unroll
    for (int i = 0; i < 16; ++i) t += acc[c][i];
  out[gid] = t;
}

// The same loop with the backward's dW-role work mix: NL8 LDS bytes per MFMA in 512-byte units
// (0, 2 = 1 KB: one 16-byte read feeding A; 3 = 1.5 KB: plus an 8-byte read feeding half of B),
// EL2 SiLU-backward elements per MFMA times two (1: half an element, as the D = 128 dW role;
// 2: one, as D = 64): s = sigmoid(z), h = z s, dz = dh (h (1 - s) + s), both rounded to bf16
// and packed, the VALU work of one activation-plane element in the dW programs. WPS waves per
// SIMD (1 or 2; the grid is WPS workgroups of four waves per CU). 16 MFMAs per iteration, four
// accumulators.
template <int NL8, int EL2, int WPS>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(WPS, WPS)))
mfma_act_mix_kernel(float* __restrict__ out, int iters) {
  __shared__ bf16x8 tile[4096];
  typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
  const unsigned gid = blockIdx.x * kThreads + threadIdx.x;
  const int lane = threadIdx.x & 63;
  for (int i = threadIdx.x; i < 4096; i += kThreads)
#pragma unroll
    for (int j = 0; j < 8; ++j) tile[i][j] = rnd_bf16(mix(blockIdx.x * 32768u + i * 8u + j));
  __syncthreads();
  bf16x8 a[16], b[16];
#pragma unroll
  for (int c = 0; c < 16; ++c)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const unsigned h = mix(gid * 256u + c * 8u + j);
      a[c][j] = rnd_bf16(h);
      b[c][j] = rnd_bf16(mix(h));
    }
  float z[8], d[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    z[q] = 0.01f * lane + q;
    d[q] = 0.5f + q;
  }
  unsigned pk = 0;
  f32x16 acc[kChains];
#pragma unroll
  for (int c = 0; c < kChains; ++c)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[c][i] = 0.f;
  constexpr int PER = EL2 >= 2 ? EL2 / 2 : 1;  // elements per activating step
  for (int it = 0; it < iters; ++it) {
    const int base = lane ^ ((it & 1) << 5);  // loop-variant, so the reads stay in the loop
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      bf16x8 A = a[s], B = b[s];
      if constexpr (NL8 >= 2) A = tile[base + s * 64];
      if constexpr (NL8 == 3) {  // index < 4096: 2048 + (at most 1023)
        const bf16x4 t = *(const bf16x4*)((const __bf16*)&tile[2048 + ((base + s * 64) & 2047)]);
        B[0] = t[0];
        B[1] = t[1];
        B[2] = t[2];
        B[3] = t[3];
      }
      acc[s % kChains] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, B, acc[s % kChains], 0, 0, 0);
      if (EL2 >= 2 || (EL2 == 1 && (s & 1) == 0)) {
#pragma unroll
        for (int q = 0; q < PER; ++q) {
          const int k = (s * PER + q) & 7;
          const float sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(z[k] * -1.4426950408889634f));
          const float h = z[k] * sg;
          const float dz = d[k] * __builtin_fmaf(h, 1.0f - sg, sg);
          const __bf16 hb = (__bf16)h, db = (__bf16)dz;
          pk ^= (unsigned)__builtin_bit_cast(unsigned short, hb) | ((unsigned)__builtin_bit_cast(unsigned short, db) << 16);
          z[k] = h;
          d[k] = dz;
        }
      }
    }
  }
  float t = (float)pk;
#pragma unroll
  for (int q = 0; q < 8; ++q) t += z[q] + d[q];
#pragma unroll
  for (int c = 0; c < kChains; ++c)
#pragma unroll
    for (int i = 0; i < 16; ++i) t += acc[c][i];
  out[gid] = t;
}

}  // namespace

// Launches `grid` workgroups of 256 threads of the dW-role work mix (mfma_act_mix_kernel) with
// `lds8` (0, 2 or 3) x 512 LDS bytes and `el2` / 2 (1 or 2) SiLU-backward elements per MFMA at
// `wps` (1 or 2) waves per SIMD; `out` holds grid * 256 floats. FLOPs = grid * 4 * iters * 16 * 32768.
extern "C" __attribute__((visibility("default"))) int fmlp_ceiling_act_mix(void* out, int iters, int lds8, int el2,
                                                                           int wps, int grid, hipStream_t stream) {
  if (out == nullptr || iters <= 0 || grid <= 0) return (int)hipErrorInvalidValue;
  float* o = (float*)out;
  const dim3 g((unsigned)grid), b(kThreads);
#define FMLP_ACT_MIX(L, E, W)                                                                   \
  if (lds8 == L && el2 == E && wps == W) {                                                      \
    hipLaunchKernelGGL((mfma_act_mix_kernel<L, E, W>), g, b, 0, stream, o, iters);              \
    return (int)hipGetLastError();                                                              \
  }
  FMLP_ACT_MIX(0, 1, 1) FMLP_ACT_MIX(0, 1, 2) FMLP_ACT_MIX(2, 1, 1) FMLP_ACT_MIX(2, 1, 2) FMLP_ACT_MIX(3, 1, 1)
  FMLP_ACT_MIX(3, 1, 2) FMLP_ACT_MIX(0, 2, 1) FMLP_ACT_MIX(0, 2, 2) FMLP_ACT_MIX(2, 2, 1) FMLP_ACT_MIX(2, 2, 2)
#undef FMLP_ACT_MIX
  return (int)hipErrorInvalidValue;
}

// Launches `grid` workgroups of 256 threads, each wave issuing iters * 16 MFMAs with
// `lds_reads` (0 or 1) LDS reads and `valu_chains` (0, 1 or 2) activation chains per MFMA;
// `out` holds grid * 256 floats. FLOPs = grid * 4 * iters * 16 * 32768.
extern "C" __attribute__((visibility("default"))) int fmlp_ceiling_mix(void* out, int iters, int lds_reads,
                                                                       int valu_chains, int grid, hipStream_t stream) {
  if (out == nullptr || iters <= 0 || grid <= 0) return (int)hipErrorInvalidValue;
  float* o = (float*)out;
  const dim3 g((unsigned)grid), b(kThreads);
  switch (lds_reads * 3 + valu_chains) {
    case 0: hipLaunchKernelGGL((mfma_mix_kernel<0, 0>), g, b, 0, stream, o, iters); break;
    case 1: hipLaunchKernelGGL((mfma_mix_kernel<0, 1>), g, b, 0, stream, o, iters); break;
    case 2: hipLaunchKernelGGL((mfma_mix_kernel<0, 2>), g, b, 0, stream, o, iters); break;
    case 3: hipLaunchKernelGGL((mfma_mix_kernel<1, 0>), g, b, 0, stream, o, iters); break;
    case 4: hipLaunchKernelGGL((mfma_mix_kernel<1, 1>), g, b, 0, stream, o, iters); break;
    case 5: hipLaunchKernelGGL((mfma_mix_kernel<1, 2>), g, b, 0, stream, o, iters); break;
    default: return (int)hipErrorInvalidValue;
  }
  return (int)hipGetLastError();
}

// Launches `grid` workgroups of 256 threads, each wave issuing iters * 4 MFMAs; `out` holds
// grid * 256 floats. Returns the hipError_t of the launch. FLOPs = grid * 4 * iters * 4 * 32768.
extern "C" __attribute__((visibility("default"))) int fmlp_ceiling_mfma(void* out, int iters, int zero_data, int grid,
                                                                        hipStream_t stream) {
  if (out == nullptr || iters <= 0 || grid <= 0) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(mfma_ceiling_kernel, dim3((unsigned)grid), dim3(kThreads), 0, stream, (float*)out, iters, zero_data);
  return (int)hipGetLastError();
}
