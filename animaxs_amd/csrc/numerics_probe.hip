// Numerical-health probes: the stats ABI of the reference's NumericalMonitor
// (NumericalMonitor.swift:21-53, 136-170, 205-212; AnimaKernels.metal:1578-1600) and its
// standalone fp16 / fp32 passes over a buffer, probe_f16_stats / probe_f32_stats
// (AnimaKernels.metal:1921-2040).  Each slot of `stats` is four uint32:
//   [0] flags: bit0 NaN, bit1 +Inf, bit2 -Inf, bit3 finite |v| > 65504;
//   [1] max |v| over the finite values, as fp32 bits (0 when there is none);
//   [2] index of the first element that set a flag, 0xFFFFFFFF when none did;
//   [3] reserved.
// A pass ORs its flags into [0] and takes the max of [1] and the min of [2] with relaxed
// device-scope atomics, so passes over several buffers accumulate into one slot until
// the slot is reset.
//
// The pass is a one-read stream: each thread walks 16-byte chunks (8 fp16 or 4 fp32
// values, four loads in flight) with a grid stride when the range is 16-byte aligned,
// element by element otherwise (256 MiB: fp16 4.9 TB/s, fp32 5.4 TB/s).  A workgroup reduces its threads' (flags, max, first) through the wave
// shuffles and 4 LDS words, and its first lane issues at most three atomics, so a pass
// of G workgroups adds at most 3G atomics to the slot's words.
#include "common.hpp"
#include "numerics_probe.hpp"

namespace anima {

constexpr int NP_THREADS = 256;
constexpr int NP_MAX_BLOCKS = 1024;
constexpr uint32_t NP_NONE = 0xffffffffu;
constexpr uint32_t NP_HALF_MAX_BITS = 0x477fe000u;   // 65504.0f

struct ProbeAcc {
  uint32_t flags, maxbits, first;
};

__device__ __forceinline__ void probe_value(float x, uint32_t i, ProbeAcc& a) {
  const uint32_t bits = __float_as_uint(x) & 0x7fffffffu;
  if (bits >= 0x7f800000u) {
    a.flags |= bits > 0x7f800000u ? 1u : (x > 0.f ? 2u : 4u);
    a.first = min(a.first, i);
  } else {
    if (bits > NP_HALF_MAX_BITS) {
      a.flags |= 8u;
      a.first = min(a.first, i);
    }
    a.maxbits = max(a.maxbits, bits);
  }
}

// fp16 on its own bits: a finite fp16 never exceeds 65504, |h| orders like its 15-bit
// pattern, and the running max (ProbeAcc::maxbits holds the 15-bit max here) is turned
// into fp32 bits once, after the loop.
__device__ __forceinline__ void probe_half_bits(uint32_t h, uint32_t i, ProbeAcc& a) {
  const uint32_t m = h & 0x7fffu;
  if (m >= 0x7c00u) {
    a.flags |= m > 0x7c00u ? 1u : ((h & 0x8000u) ? 4u : 2u);
    a.first = min(a.first, i);
  } else {
    a.maxbits = max(a.maxbits, m);
  }
}

template <typename T>
__device__ __forceinline__ void probe_chunk(const u32x4& raw, uint32_t i0, ProbeAcc& a) {
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      probe_half_bits(raw[e] & 0xffffu, i0 + 2 * e, a);
      probe_half_bits(raw[e] >> 16, i0 + 2 * e + 1, a);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) probe_value(__uint_as_float(raw[e]), i0 + e, a);
  }
}

template <typename T>
__global__ __launch_bounds__(NP_THREADS) void numerics_probe_kernel(const T* v, uint32_t count, int vec,
                                                                   uint32_t* slot) {
  ProbeAcc a{0u, 0u, NP_NONE};
  // 64-bit loop counters: with count close to 2^32 a 32-bit i + stride would wrap.
  const uint64_t stride = (uint64_t)gridDim.x * NP_THREADS;
  const uint64_t t0 = (uint64_t)blockIdx.x * NP_THREADS + threadIdx.x;
  uint64_t scalar_from = 0;
  if (vec) {
    constexpr uint32_t EPV = 16 / sizeof(T);
    const uint64_t nvec = count / EPV;
    const u32x4* src = reinterpret_cast<const u32x4*>(v);
    // Four chunks in flight per thread before any is examined.
    uint64_t c = t0;
    for (; c + 3 * stride < nvec; c += 4 * stride) {
      u32x4 r[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) r[u] = __builtin_nontemporal_load(src + c + u * stride);
#pragma unroll
      for (int u = 0; u < 4; ++u) probe_chunk<T>(r[u], (uint32_t)((c + u * stride) * EPV), a);
    }
    for (; c < nvec; c += stride) probe_chunk<T>(__builtin_nontemporal_load(src + c), (uint32_t)(c * EPV), a);
    scalar_from = nvec * EPV;
  }
  for (uint64_t i = scalar_from + t0; i < count; i += stride) {
    if constexpr (sizeof(T) == 2)
      probe_half_bits(__builtin_bit_cast(uint16_t, v[i]), (uint32_t)i, a);
    else
      probe_value(v[i], (uint32_t)i, a);
  }
  if constexpr (sizeof(T) == 2)   // the 15-bit fp16 magnitude as fp32 bits (0 stays 0)
    a.maxbits = __float_as_uint((float)__builtin_bit_cast(half_t, (uint16_t)a.maxbits));

#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    a.flags |= (uint32_t)__shfl_xor((int)a.flags, m, 64);
    a.maxbits = max(a.maxbits, (uint32_t)__shfl_xor((int)a.maxbits, m, 64));
    a.first = min(a.first, (uint32_t)__shfl_xor((int)a.first, m, 64));
  }
  __shared__ uint32_t red[3][NP_THREADS / 64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) {
    red[0][wave] = a.flags;
    red[1][wave] = a.maxbits;
    red[2][wave] = a.first;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 1; w < NP_THREADS / 64; ++w) {
      a.flags |= red[0][w];
      a.maxbits = max(a.maxbits, red[1][w]);
      a.first = min(a.first, red[2][w]);
    }
    if (a.flags != 0u) {
      __hip_atomic_fetch_or(slot + 0, a.flags, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_fetch_min(slot + 2, a.first, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (a.maxbits != 0u) __hip_atomic_fetch_max(slot + 1, a.maxbits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Slot reset (the monitor's beginRun, NumericalMonitor.swift:205-212): flags, max and
// the reserved word 0, first index 0xFFFFFFFF.  A kernel rather than a memset, so that
// a caller may record it in a HIP graph.
// 64-bit word indices: slots up to 2^31 - 1 make up to 2^33 words.
__global__ __launch_bounds__(NP_THREADS) void numerics_probe_reset_kernel(uint32_t* stats, uint64_t words) {
  const uint64_t i = (uint64_t)blockIdx.x * NP_THREADS + threadIdx.x;
  if (i < words) stats[i] = (i & 3u) == 2u ? NP_NONE : 0u;
}

void launch_numerics_probe(const void* values, int64_t count, bool f16, uint32_t* slot, hipStream_t stream) {
  if (count <= 0) return;
  const bool vec = (reinterpret_cast<uintptr_t>(values) & 15u) == 0;
  const int64_t units = vec ? count / (f16 ? 8 : 4) : count;
  int64_t blocks = (units + NP_THREADS - 1) / NP_THREADS;
  blocks = blocks < 1 ? 1 : (blocks > NP_MAX_BLOCKS ? NP_MAX_BLOCKS : blocks);
  if (f16)
    hipLaunchKernelGGL(numerics_probe_kernel<half_t>, dim3((unsigned)blocks), dim3(NP_THREADS), 0, stream,
                       static_cast<const half_t*>(values), (uint32_t)count, (int)vec, slot);
  else
    hipLaunchKernelGGL(numerics_probe_kernel<float>, dim3((unsigned)blocks), dim3(NP_THREADS), 0, stream,
                       static_cast<const float*>(values), (uint32_t)count, (int)vec, slot);
  ANIMA_HIP(hipGetLastError());
}

void launch_numerics_probe_reset(uint32_t* stats, int64_t slots, hipStream_t stream) {
  if (slots <= 0) return;
  const int64_t words = slots * NUMERICS_PROBE_SLOT_UINTS;
  const int64_t blocks = (words + NP_THREADS - 1) / NP_THREADS;
  hipLaunchKernelGGL(numerics_probe_reset_kernel, dim3((unsigned)blocks), dim3(NP_THREADS), 0, stream, stats,
                     (uint64_t)words);
  ANIMA_HIP(hipGetLastError());
}

}  // namespace anima
