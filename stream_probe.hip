// Streaming-bandwidth reference for bench.py (measurement only: not part of the operator
// library or its C ABI, built into its own libictc_stream_probe.so).
//
// A plain grid-stride kernel that moves a fixed read:write byte mix with float4 accesses:
// per unit it reads R float4 (one from each of R contiguous read streams) and writes W
// float4 (one to each of W write streams).  Timing it at the byte count and mix of a hot
// kernel gives the bandwidth an ideal streaming kernel reaches for that traffic on this
// GPU, the practical ceiling beside the 8 TB/s datasheet peak.  Loads use the default or
// the non-temporal cache policy (NT): callers take the better of the two.
//
// A second probe measures the fp32 vector (VALU) FMA rate this build can reach: every lane
// runs 16 independent fma chains on registers (scalar v_fma/v_fmac: the library is compiled
// without packed FP32, so no v_pk_fma_f32 can appear) and writes one float, so the work is
// 32 FLOPs per lane per iteration and memory traffic is negligible.
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

// VGPR_B: acc += b * c with b, c per-lane register values (v_fmac_f32, the VOP2 form with the
// accumulator as addend and every operand in a VGPR) rather than acc = acc * b + c with b, c
// kernel arguments in SGPRs (v_fma_f32, VOP3).
template <bool VGPR_B>
__global__ void __launch_bounds__(256) valu_fma_kernel(float* __restrict__ out, int iters, float b, float c) {
  float acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = static_cast<float>(threadIdx.x + i);
  const float bv = VGPR_B ? b + 1e-7f * static_cast<float>(threadIdx.x & 1) : b;
  const float cv = VGPR_B ? c * static_cast<float>(1 + (threadIdx.x & 1)) : c;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = VGPR_B ? __builtin_fmaf(bv, cv, acc[i]) : __builtin_fmaf(acc[i], bv, cv);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s += acc[i];
  out[blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x] = s;
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

// fp32 FMA throughput: grid blocks of 256 lanes, each lane 16 chains x iters fmas
// (32 * iters FLOPs per lane); out must hold grid * 256 floats.  vgpr_operands != 0 keeps
// every fma operand in a VGPR.  Returns 0 or -1.
extern "C" int ictc_probe_valu_fma(void* out, int iters, int grid, int vgpr_operands, hipStream_t stream) {
  if (out == nullptr || iters <= 0 || grid <= 0) return -1;
  if (vgpr_operands)
    hipLaunchKernelGGL(valu_fma_kernel<true>, dim3(grid), dim3(256), 0, stream, static_cast<float*>(out), iters,
                       0.999f, 1e-3f);
  else
    hipLaunchKernelGGL(valu_fma_kernel<false>, dim3(grid), dim3(256), 0, stream, static_cast<float*>(out), iters,
                       0.999f, 1e-3f);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}
