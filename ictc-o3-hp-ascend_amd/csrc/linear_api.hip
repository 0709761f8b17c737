// Per-degree channel linear on fp32 MFMA (gfx950): the path-preserving message linear of the
// MACE interaction (reference mace_ictc/models/pure_cartesian_ictd_fix.py:629-661,
// PathPreservingLinearSO3; native route ictc_o3/ascendc/linear.py:12-136), applied straight to
// the message kernel's packed output and writing the mul_ir node layout.
//
// Per degree l (d = 2l + 1, K_l = counts[l] * C):
//   x  row n, degree block l:  [counts[l]][d][C]          (ir_mul, the message output)
//   y  row n, degree block l:  [O][d]                     (mul_ir, offset O * l^2)
//   forward:     y[n, o, m]            = alpha * sum_{k, c} W_l[o, k C + c] x[n, k, m, c]
//   input grad:  gx[n, k, m, c]        = alpha * sum_o gy[n, o, m] W_l[o, k C + c]
//   mul_ir map:  y[n, o, m]            = alpha * sum_c W_l[o, c] x[n, c, m]   (counts all 1; x
//                                        mul_ir [N, C (L+1)^2], per degree [C][d] at offset C l^2)
// i.e. for the rows rho = n d + m, Y = alpha X W^T and gX = alpha gY W, one GEMM per degree with
// the layout changes folded into the tile loads and stores (no transposed copies, no
// concatenation, the 1/avg_num_neighbors scale as alpha).
//
// Tiling: a 256-thread block computes a 64-row x 64-column output tile of one degree (grid.z);
// K is walked in chunks of 32 staged through LDS, then each wave runs v_mfma_f32_16x16x4_f32 over
// its 16 rows and the tile's 4 column tiles.  Operand layout of that instruction: lane l supplies
// A[l % 16][k_l] and B[k_l][l % 16] and receives D[4 (l / 16) + v][l % 16], v = 0..3, where k_l is
// the instruction's k index l / 16.  Which actual k a lane feeds is free as long as A and B agree:
// here four consecutive MFMAs j = 0..3 cover a 16-wide k group with k = 4 (l / 16) + j, so each
// lane reads its four A (and B) values of a group with one 16-byte LDS read.  Every sum runs in a
// fixed order (bit-identical run to run).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ictc_hip.h"

namespace ictc {
namespace {

constexpr int kTile = 64;   // rows and columns per block
constexpr int kKc = 32;     // K per LDS chunk
constexpr int kPitch = kKc + 4;   // LDS row pitch in floats (16-byte aligned rows)

typedef float f32x4_t __attribute__((ext_vector_type(4)));

struct DegreeGeometry {
  int64_t rows;       // N d
  int d;              // 2l + 1
  int k;              // counts[l] * C
  int64_t xoff;       // first float of the degree block in an x row
  int64_t yoff;       // first float of the degree block in a y row
  const float* w;     // [O, k]
};

struct LinearArgs {
  DegreeGeometry g[ICTC_LINEAR_MAX_DEGREES];
  int64_t xwidth, ywidth;
  int channels, out_channels;
  float alpha;
};

// MODE kForward: A = x rows (K = x columns), B^T = W rows, D -> y.  kInputGrad: A = gy rows
// (K = O), B = W, D -> gx columns.  kMulIr: A = mul_ir x rows (K = C, stride d), B^T = W rows,
// D -> y (mul_ir).  VEC (channels a multiple of 32): each 32-wide K chunk of an x row lies in one
// path block and weight rows are float4-aligned, so operands are fetched into registers one chunk
// ahead (their loads in flight while the MFMAs of the current chunk run); with two LDS buffers
// (NBUF 2) the next chunk is staged into the other buffer right after those MFMAs (one barrier per
// chunk), with one (NBUF 1, half the LDS and so twice the resident blocks) after a second barrier.
// The forward's long K (counts C) takes two buffers, the input adjoint's short K (O) one.
// Without VEC, element by element, one chunk at a time.
enum LinearMode { kForward = 0, kInputGrad = 1, kMulIr = 2 };

template <int MODE, bool VEC, int NBUF>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NBUF == 1 ? 8 : 4)))
degree_linear_kernel(const float* __restrict__ in, float* __restrict__ out, const LinearArgs a) {
  constexpr bool FWD = MODE != kInputGrad;      // D -> mul_ir y rows, B^T = W rows
  constexpr bool STRIDED = MODE != kForward;    // A rows read at stride d over K (mul_ir)
  const DegreeGeometry& g = a.g[blockIdx.z];
  const int ncols = FWD ? a.out_channels : g.k;   // output columns
  const int kdim = FWD ? g.k : a.out_channels;    // reduction length
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kTile;
  const int c0 = blockIdx.y * kTile;
  // uniform per block; a degree without path blocks (kdim 0) writes its zero forward rows
  if (r0 >= g.rows || c0 >= ncols) return;
  __shared__ __align__(16) float sA[NBUF][kTile][kPitch];   // [buffer][row][k]
  __shared__ __align__(16) float sB[NBUF][kTile][kPitch];   // [buffer][column][k]
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int C = a.channels;
  // A staging: thread t holds 8 consecutive k of tile row t / 4
  const int ar = tid >> 2, akq = (tid & 3) * 8;
  const int64_t arho = r0 + ar;
  const bool arow = arho < g.rows;
  const int64_t an = arow ? arho / g.d : 0;
  const int am = arow ? static_cast<int>(arho - an * g.d) : 0;
  const float* __restrict__ abase = MODE == kForward   ? in + an * a.xwidth + g.xoff + static_cast<int64_t>(am) * C
                                    : MODE == kInputGrad ? in + an * a.ywidth + g.yoff + am
                                                         : in + an * a.xwidth + g.xoff + am;
  // !FWD B staging: thread t holds weight row k0 + t / 8, columns c0 + 8 (t % 8) .. + 7 (two
  // float4 loads), stored transposed element by element.  The k index of B column col is
  // XOR-swizzled by bsw(col) (a multiple of 8 below 32, so every aligned 4-group of k stays
  // contiguous and in its row): the transposed stores of a wave then meet at most two lanes per
  // bank, and with the 36-float pitch the 16-byte MFMA operand reads stay conflict-free.
  const int wk = tid >> 3, wc = (tid & 7) * 8;
  auto bsw = [](int col) { return FWD ? 0 : ((col >> 3) & 3) * 8; };
  f32x4_t acc[4] = {};
  const int fr = lane & 15, fq = (lane >> 4) * 4;
  auto mfma_chunk = [&](int buf) {
#pragma unroll
    for (int kg = 0; kg < kKc; kg += 16) {
      const f32x4_t av = *reinterpret_cast<const f32x4_t*>(&sA[buf][wave * 16 + fr][kg + fq]);
      if constexpr (NBUF == 1) {
        // one B operand live at a time (the register budget of 8 waves per SIMD); the
        // accumulation chains of the other resident waves fill the MFMA pipe
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const f32x4_t bv = *reinterpret_cast<const f32x4_t*>(&sB[buf][t * 16 + fr][(kg + fq) ^ bsw(t * 16 + fr)]);
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j], bv[j], acc[t], 0, 0, 0);
        }
      } else {
        f32x4_t bv[4];
#pragma unroll
        for (int t = 0; t < 4; ++t)
          bv[t] = *reinterpret_cast<const f32x4_t*>(&sB[buf][t * 16 + fr][(kg + fq) ^ bsw(t * 16 + fr)]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
          for (int t = 0; t < 4; ++t) acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j], bv[t][j], acc[t], 0, 0, 0);
        }
      }
    }
  };
  if constexpr (VEC) {
    // registers of one chunk: A (8 floats of the thread's row), B (8 floats)
    f32x4_t ra0, ra1, rb0, rb1;
    auto fetch = [&](int k0) {
      const bool kin = k0 + akq < kdim;
      ra0 = f32x4_t{};
      ra1 = f32x4_t{};
      rb0 = f32x4_t{};
      rb1 = f32x4_t{};
      if constexpr (STRIDED) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {   // mul_ir row: stride d over K
          if (arow && k0 + akq + u < kdim) ra0[u] = abase[static_cast<int64_t>(k0 + akq + u) * g.d];
          if (arow && k0 + akq + 4 + u < kdim) ra1[u] = abase[static_cast<int64_t>(k0 + akq + 4 + u) * g.d];
        }
      } else {
        const int blk = k0 / C, c = k0 - blk * C + akq;
        if (arow && kin) {
          const float* p = abase + static_cast<int64_t>(blk) * g.d * C + c;
          ra0 = *reinterpret_cast<const f32x4_t*>(p);
          ra1 = *reinterpret_cast<const f32x4_t*>(p + 4);
        }
      }
      if constexpr (FWD) {
        const int col = c0 + ar;   // weight row col, 8 consecutive k
        if (col < ncols && kin) {
          const float* p = g.w + static_cast<int64_t>(col) * g.k + k0 + akq;
          rb0 = *reinterpret_cast<const f32x4_t*>(p);
          rb1 = *reinterpret_cast<const f32x4_t*>(p + 4);
        }
      } else {
        const int kk = k0 + wk;
        if (kk < kdim && c0 + wc < ncols) {   // ncols (counts C) is a multiple of 32
          const float* p = g.w + static_cast<int64_t>(kk) * g.k + c0 + wc;
          rb0 = *reinterpret_cast<const f32x4_t*>(p);
          rb1 = *reinterpret_cast<const f32x4_t*>(p + 4);
        }
      }
    };
    auto stage = [&](int buf) {
      *reinterpret_cast<f32x4_t*>(&sA[buf][ar][akq]) = ra0;
      *reinterpret_cast<f32x4_t*>(&sA[buf][ar][akq + 4]) = ra1;
      if constexpr (FWD) {
        *reinterpret_cast<f32x4_t*>(&sB[buf][ar][akq]) = rb0;
        *reinterpret_cast<f32x4_t*>(&sB[buf][ar][akq + 4]) = rb1;
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          sB[buf][wc + u][wk ^ bsw(wc + u)] = rb0[u];
          sB[buf][wc + 4 + u][wk ^ bsw(wc + 4 + u)] = rb1[u];
        }
      }
    };
    fetch(0);
    if constexpr (NBUF == 2) {
      // buffer c & 1 holds chunk c; chunk c + 1 is fetched before and staged after chunk c's
      // MFMAs, into the buffer every wave finished reading at the previous barrier
      stage(0);
      __syncthreads();
      int buf = 0;
      for (int k0 = 0; k0 < kdim; k0 += kKc) {
        const bool more = k0 + kKc < kdim;
        if (more) fetch(k0 + kKc);
        mfma_chunk(buf);
        if (more) stage(buf ^ 1);
        __syncthreads();
        buf ^= 1;
      }
    } else {
      for (int k0 = 0; k0 < kdim; k0 += kKc) {
        stage(0);
        __syncthreads();
        if (k0 + kKc < kdim) fetch(k0 + kKc);
        mfma_chunk(0);
        __syncthreads();
      }
    }
  } else {
    for (int k0 = 0; k0 < kdim; k0 += kKc) {
      if constexpr (FWD) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int kk = k0 + akq + u;
          float v = 0.f;
          if (arow && kk < kdim) {
            if constexpr (STRIDED) {
              v = abase[static_cast<int64_t>(kk) * g.d];
            } else {
              const int blk = kk / C, c = kk - blk * C;
              v = abase[static_cast<int64_t>(blk) * g.d * C + c];
            }
          }
          sA[0][ar][akq + u] = v;
          const int col = c0 + ar;
          sB[0][ar][akq + u] = (col < ncols && kk < kdim) ? g.w[static_cast<int64_t>(col) * g.k + kk] : 0.f;
        }
      } else {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int kk = k0 + akq + u;
          sA[0][ar][akq + u] = (arow && kk < kdim) ? abase[static_cast<int64_t>(kk) * g.d] : 0.f;
        }
        const int kk = k0 + wk;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int col = c0 + wc + u;
          sB[0][wc + u][wk ^ bsw(wc + u)] =
              (kk < kdim && col < ncols) ? g.w[static_cast<int64_t>(kk) * g.k + col] : 0.f;
        }
      }
      __syncthreads();
      mfma_chunk(0);
      __syncthreads();
    }
  }
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int64_t rho = r0 + wave * 16 + 4 * (lane >> 4) + v;
    if (rho >= g.rows) continue;
    const int64_t n = rho / g.d;
    const int m = static_cast<int>(rho - n * g.d);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int col = c0 + t * 16 + (lane & 15);
      if (col >= ncols) continue;
      const float val = a.alpha * acc[t][v];
      if (FWD) {
        out[n * a.ywidth + g.yoff + static_cast<int64_t>(col) * g.d + m] = val;
      } else {
        const int blk = col / C, c = col - blk * C;
        out[n * a.xwidth + g.xoff + (static_cast<int64_t>(blk) * g.d + m) * C + c] = val;
      }
    }
  }
}

int prepare(const ictc_degree_linear_desc* desc, const float* const* weights, float alpha, int64_t nodes,
            LinearArgs* a, int* live_degrees, int64_t* max_rows, int* max_cols, bool fwd) {
  if (desc == nullptr || weights == nullptr || nodes < 0) return ICTC_ERR_INVALID_ARGUMENT;
  if (desc->lmax < 0 || desc->lmax >= ICTC_LINEAR_MAX_DEGREES || desc->channels < 1 || desc->out_channels < 1)
    return ICTC_ERR_INVALID_ARGUMENT;
  int64_t xw = 0;
  for (int l = 0; l <= desc->lmax; ++l) {
    if (desc->counts[l] < 0) return ICTC_ERR_INVALID_ARGUMENT;
    xw += static_cast<int64_t>(desc->counts[l]) * (2 * l + 1) * desc->channels;
  }
  a->xwidth = xw;
  a->ywidth = static_cast<int64_t>(desc->out_channels) * (desc->lmax + 1) * (desc->lmax + 1);
  a->channels = desc->channels;
  a->out_channels = desc->out_channels;
  a->alpha = alpha;
  *live_degrees = desc->lmax + 1;
  *max_rows = 0;
  *max_cols = 0;
  int64_t xoff = 0;
  for (int l = 0; l <= desc->lmax; ++l) {
    DegreeGeometry& g = a->g[l];
    g.d = 2 * l + 1;
    g.rows = nodes * g.d;
    g.k = desc->counts[l] * desc->channels;
    g.xoff = xoff;
    g.yoff = static_cast<int64_t>(desc->out_channels) * l * l;
    g.w = weights[l];
    if (g.k > 0 && g.w == nullptr) return ICTC_ERR_INVALID_ARGUMENT;
    xoff += static_cast<int64_t>(g.k) * g.d;
    if (g.rows > *max_rows) *max_rows = g.rows;
    const int cols = fwd ? desc->out_channels : g.k;
    if (cols > *max_cols) *max_cols = cols;
  }
  return ICTC_OK;
}

template <int MODE>
int launch(const ictc_degree_linear_desc* desc, const float* in, const float* const* weights, float alpha,
           float* out, int64_t nodes, hipStream_t stream) {
  LinearArgs a{};
  int degrees = 0, max_cols = 0;
  int64_t max_rows = 0;
  const int st = prepare(desc, weights, alpha, nodes, &a, &degrees, &max_rows, &max_cols, MODE != kInputGrad);
  if (st != ICTC_OK) return st;
  if (MODE == kMulIr) {   // one channel block per degree: x mul_ir [N, C (L+1)^2]
    for (int l = 0; l <= desc->lmax; ++l)
      if (desc->counts[l] != 1) return ICTC_ERR_INVALID_ARGUMENT;
  }
  if (nodes == 0) return ICTC_OK;
  if (in == nullptr || out == nullptr) return ICTC_ERR_INVALID_ARGUMENT;
  const int64_t row_tiles = (max_rows + kTile - 1) / kTile;
  if (row_tiles > 0x7fffffff) return ICTC_ERR_UNSUPPORTED;
  const dim3 grid(static_cast<unsigned>(row_tiles), static_cast<unsigned>((max_cols + kTile - 1) / kTile),
                  static_cast<unsigned>(degrees));
  // two LDS buffers for the long K of the forward (counts C), one for the short K of the others
  if (desc->channels % 32 == 0)
    hipLaunchKernelGGL((degree_linear_kernel<MODE, true, MODE == kForward ? 2 : 1>), grid, dim3(256), 0, stream, in,
                       out, a);
  else
    hipLaunchKernelGGL((degree_linear_kernel<MODE, false, 1>), grid, dim3(256), 0, stream, in, out, a);
  return hipGetLastError() == hipSuccess ? ICTC_OK : ICTC_ERR_LAUNCH;
}

}  // namespace
}  // namespace ictc

extern "C" {

int ictc_hip_degree_linear_forward(const ictc_degree_linear_desc* desc, const float* x, const float* const* weights,
                                   float alpha, float* y, int64_t nodes, hipStream_t stream) {
  return ictc::launch<ictc::kForward>(desc, x, weights, alpha, y, nodes, stream);
}

int ictc_hip_degree_linear_input_grad(const ictc_degree_linear_desc* desc, const float* grad_y,
                                      const float* const* weights, float alpha, float* grad_x, int64_t nodes,
                                      hipStream_t stream) {
  return ictc::launch<ictc::kInputGrad>(desc, grad_y, weights, alpha, grad_x, nodes, stream);
}

int ictc_hip_degree_linear_mul_ir(const ictc_degree_linear_desc* desc, const float* x, const float* const* weights,
                                  float alpha, float* y, int64_t nodes, hipStream_t stream) {
  return ictc::launch<ictc::kMulIr>(desc, x, weights, alpha, y, nodes, stream);
}

}  // extern "C"
