// Streaming-bandwidth reference for bench.py (measurement only: not part of the operator
// library or its C ABI, built into its own libictc_stream_probe.so).
//
// A plain grid-stride kernel that moves a fixed read:write byte mix with float4 accesses:
// per unit it reads R float4 (one from each of R contiguous read streams) and writes W
// float4 (one to each of W write streams).  Timing it at the byte count and mix of a hot
// kernel gives the bandwidth an ideal streaming kernel reaches for that traffic on this
// GPU, the practical ceiling beside the 8 TB/s datasheet peak.  Loads use the default or
// the non-temporal cache policy (NT): callers take the better of the two.
#include <hip/hip_runtime.h>
#include <stddef.h>

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

template <int R, int W, bool NT>
__global__ void __launch_bounds__(256) stream_mix_kernel(const f4* __restrict__ a, f4* __restrict__ b, size_t units) {
  for (size_t u = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; u < units;
       u += static_cast<size_t>(gridDim.x) * blockDim.x) {
    f4 v[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const f4* src = a + static_cast<size_t>(r) * units + u;
      v[r] = NT ? __builtin_nontemporal_load(src) : *src;
    }
    f4 acc = v[0];
#pragma unroll
    for (int r = 1; r < R; ++r) acc += v[r];
#pragma unroll
    for (int w = 0; w < W; ++w) __builtin_nontemporal_store(acc * static_cast<float>(w + 1), b + static_cast<size_t>(w) * units + u);
  }
}

template <int R, int W, bool NT>
int launch(const void* a, void* b, size_t units, int grid, hipStream_t stream) {
  hipLaunchKernelGGL((stream_mix_kernel<R, W, NT>), dim3(grid), dim3(256), 0, stream, static_cast<const f4*>(a),
                     static_cast<f4*>(b), units);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace

// Units of the (reads, writes) mix: unit u reads a[r * units + u] for r < reads and writes
// b[w * units + u] for w < writes (float4 elements), so a must hold reads * units and b
// writes * units float4.  Supported mixes: (7, 2) and (2, 5); nt_loads != 0 selects
// non-temporal loads.  Returns 0, or -1 on an unsupported mix, bad arguments or a launch error.
extern "C" int ictc_probe_stream_mix(int reads, int writes, int nt_loads, const void* a, void* b, size_t units,
                                     int grid, hipStream_t stream) {
  if (a == nullptr || b == nullptr || units == 0 || grid <= 0) return -1;
  if (reads == 7 && writes == 2)
    return nt_loads ? launch<7, 2, true>(a, b, units, grid, stream) : launch<7, 2, false>(a, b, units, grid, stream);
  if (reads == 2 && writes == 5)
    return nt_loads ? launch<2, 5, true>(a, b, units, grid, stream) : launch<2, 5, false>(a, b, units, grid, stream);
  return -1;
}
