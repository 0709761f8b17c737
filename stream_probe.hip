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
// 32 FLOPs per lane per iteration and memory traffic is negligible.  A third gives the issue
// cost of individual VALU instruction forms (operand kinds and encodings).
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

// Issue cost of one VALU instruction form: every lane runs 16 independent chains of that
// instruction (inline asm, so the form is exactly the one named), iters times.  Forms:
//   0 v_fmac_f32_e32 v, v, v      (VOP2, all operands VGPRs)
//   1 v_fmac_f32_e32 v, literal, v
//   2 v_fma_f32 v, v, v, v        (VOP3, all VGPRs, destination distinct from the addend)
//   3 v_fmac_f32_e32 v, s, v      (an SGPR operand)
//   4 v_fmac_f32_e64 v, v, v      (the VOP3 encoding of fmac)
//   5 v_fmac_f32_dpp v, v, v      (a DPP lane permutation)
//   6 v_cndmask_b32_e64 v, v, v, s[..]   (a lane mask in an SGPR pair)
//   7 v_readlane_b32 s, v, 1
template <int FORM>
__global__ void __launch_bounds__(256) valu_form_kernel(float* __restrict__ out, int iters, float b, float c) {
  float a[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) a[i] = static_cast<float>(threadIdx.x + i);
  const float vb = b + 1e-7f * static_cast<float>(threadIdx.x & 1);
  const float vc = c * static_cast<float>(1 + (threadIdx.x & 1));
  const unsigned long long mask = __ballot(threadIdx.x & 1);
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if constexpr (FORM == 0) asm volatile("v_fmac_f32_e32 %0, %1, %2" : "+v"(a[i]) : "v"(vb), "v"(vc));
      if constexpr (FORM == 1) asm volatile("v_fmac_f32_e32 %0, 0x3f7fbe77, %1" : "+v"(a[i]) : "v"(vc));
      if constexpr (FORM == 2) asm volatile("v_fma_f32 %0, %1, %2, %3" : "=v"(a[i]) : "v"(vb), "v"(vc), "v"(a[(i + 1) & 15]));
      if constexpr (FORM == 3) asm volatile("v_fmac_f32_e32 %0, %1, %2" : "+v"(a[i]) : "s"(b), "v"(vc));
      if constexpr (FORM == 4) asm volatile("v_fmac_f32_e64 %0, %1, %2" : "+v"(a[i]) : "v"(vb), "v"(vc));
      if constexpr (FORM == 5)
        asm volatile("v_fmac_f32_dpp %0, %1, %2 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf" : "+v"(a[i]) : "v"(vb), "v"(vc));
      if constexpr (FORM == 6) asm volatile("v_cndmask_b32_e64 %0, %0, %1, %2" : "+v"(a[i]) : "v"(vb), "s"(mask));
      if constexpr (FORM == 7) asm volatile("v_readlane_b32 s0, %0, 1" ::"v"(a[i]) : "s0");
    }
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s += a[i];
  out[blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x] = s;
}

// Issue rate of one wave: CHAINS independent v_fmac_f32 chains (16 instructions per iteration in
// total) in blocks of 256 lanes whose dynamic LDS allocation limits residency to a chosen number of
// blocks per CU, i.e. waves per SIMD.
template <int CHAINS>
__global__ void __launch_bounds__(256) valu_chain_kernel(float* __restrict__ out, int iters, float b, float c) {
  extern __shared__ float pad[];
  float a[CHAINS];
#pragma unroll
  for (int i = 0; i < CHAINS; ++i) a[i] = static_cast<float>(threadIdx.x + i);
  const float vb = b + 1e-7f * static_cast<float>(threadIdx.x & 1);
  const float vc = c * static_cast<float>(1 + (threadIdx.x & 1));
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int r = 0; r < 16 / CHAINS; ++r) {
#pragma unroll
      for (int k = 0; k < CHAINS; ++k) asm volatile("v_fmac_f32_e32 %0, %1, %2" : "+v"(a[k]) : "v"(vb), "v"(vc));
    }
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < CHAINS; ++i) s += a[i];
  if (threadIdx.x == 0) pad[0] = s;
  __syncthreads();
  out[blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x] = s + pad[threadIdx.x & 1];
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

// Issue cost of VALU instruction form `form` (valu_form_kernel above): grid blocks of 256 lanes,
// 16 instructions x iters per lane; out must hold grid * 256 floats.  Returns 0 or -1.
extern "C" int ictc_probe_valu_form(void* out, int form, int iters, int grid, hipStream_t stream) {
  if (out == nullptr || iters <= 0 || grid <= 0) return -1;
  float* o = static_cast<float*>(out);
  switch (form) {
    case 0: hipLaunchKernelGGL(valu_form_kernel<0>, dim3(grid), dim3(256), 0, stream, o, iters, 0.999f, 1e-3f); break;
    case 1: hipLaunchKernelGGL(valu_form_kernel<1>, dim3(grid), dim3(256), 0, stream, o, iters, 0.999f, 1e-3f); break;
    case 2: hipLaunchKernelGGL(valu_form_kernel<2>, dim3(grid), dim3(256), 0, stream, o, iters, 0.999f, 1e-3f); break;
    case 3: hipLaunchKernelGGL(valu_form_kernel<3>, dim3(grid), dim3(256), 0, stream, o, iters, 0.999f, 1e-3f); break;
    case 4: hipLaunchKernelGGL(valu_form_kernel<4>, dim3(grid), dim3(256), 0, stream, o, iters, 0.999f, 1e-3f); break;
    case 5: hipLaunchKernelGGL(valu_form_kernel<5>, dim3(grid), dim3(256), 0, stream, o, iters, 0.999f, 1e-3f); break;
    case 6: hipLaunchKernelGGL(valu_form_kernel<6>, dim3(grid), dim3(256), 0, stream, o, iters, 0.999f, 1e-3f); break;
    case 7: hipLaunchKernelGGL(valu_form_kernel<7>, dim3(grid), dim3(256), 0, stream, o, iters, 0.999f, 1e-3f); break;
    default: return -1;
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// One wave's issue rate: chains (1, 2, 4 or 8) independent FMA chains, waves_per_simd (1, 2 or 4)
// resident waves per SIMD (blocks per CU limited through their LDS allocation), cus * waves_per_simd
// blocks of 256 lanes, 16 instructions x iters per lane; out must hold that many blocks x 256
// floats.  Returns 0 or -1.
extern "C" int ictc_probe_valu_chains(void* out, int chains, int waves_per_simd, int cus, int iters,
                                      hipStream_t stream) {
  if (out == nullptr || iters <= 0 || cus <= 0) return -1;
  if (waves_per_simd != 1 && waves_per_simd != 2 && waves_per_simd != 4) return -1;
  const size_t lds = (160u * 1024u) / static_cast<unsigned>(waves_per_simd) - 1024u;
  const dim3 grid(static_cast<unsigned>(cus * waves_per_simd));
  float* o = static_cast<float*>(out);
  switch (chains) {
    case 1: hipLaunchKernelGGL(valu_chain_kernel<1>, grid, dim3(256), lds, stream, o, iters, 0.999f, 1e-3f); break;
    case 2: hipLaunchKernelGGL(valu_chain_kernel<2>, grid, dim3(256), lds, stream, o, iters, 0.999f, 1e-3f); break;
    case 4: hipLaunchKernelGGL(valu_chain_kernel<4>, grid, dim3(256), lds, stream, o, iters, 0.999f, 1e-3f); break;
    case 8: hipLaunchKernelGGL(valu_chain_kernel<8>, grid, dim3(256), lds, stream, o, iters, 0.999f, 1e-3f); break;
    default: return -1;
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}
