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

constexpr int kTile = 64;   // rows per block, and columns per block of the forward modes
constexpr int kTileIg = 128;   // columns per block of the input adjoint
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
// D -> y (mul_ir).  VEC (channels, and for kInputGrad out_channels, multiples of 32): every
// 32-wide K chunk is full, each K chunk of an x row lies in one path block and weight rows are
// float4-aligned, so operands are fetched into registers one chunk ahead (their loads in flight
// while the MFMAs of the current chunk run); with two LDS buffers
// (NBUF 2) the next chunk is staged into the other buffer right after those MFMAs (one barrier per
// chunk), with one (NBUF 1, half the LDS and so twice the resident blocks) after a second barrier.
// The forward's long K (counts C) takes two buffers, the input adjoint's short K (O) one.
// Without VEC, element by element, one chunk at a time.
enum LinearMode { kForward = 0, kInputGrad = 1, kMulIr = 2 };

template <int MODE, bool VEC, int NBUF, int TN>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NBUF == 1 ? (TN > kTile ? 5 : 8) : 4)))
degree_linear_kernel(const float* __restrict__ in, float* __restrict__ out, const LinearArgs a) {
  constexpr bool FWD = MODE != kInputGrad;      // D -> mul_ir y rows, B^T = W rows
  constexpr int NT = TN / 16;                   // 16-column MFMA tiles per wave
  static_assert(FWD ? TN == kTile : (TN == kTile || TN == kTileIg), "column tile");
  constexpr bool STRIDED = MODE != kForward;    // A rows read at stride d over K (mul_ir)
  // the degree's geometry in registers (read once from the kernel arguments)
  const DegreeGeometry g = a.g[blockIdx.z];
  const int d = g.d;
  const int ncols = FWD ? a.out_channels : g.k;   // output columns
  const int kdim = FWD ? g.k : a.out_channels;    // reduction length
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kTile;
  const int c0 = blockIdx.y * TN;
  // uniform per block; a degree without path blocks (kdim 0) writes its zero forward rows
  if (r0 >= g.rows || c0 >= ncols) return;
  __shared__ __align__(16) float sA[NBUF][kTile][kPitch];   // [buffer][row][k]
  __shared__ __align__(16) float sB[NBUF][TN][kPitch];      // [buffer][column][k]
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int C = a.channels;
  // A staging: thread t holds 8 consecutive k of tile row t / 4
  const int ar = tid >> 2, akq = (tid & 3) * 8;
  const int64_t arho = r0 + ar;
  const bool arow = arho < g.rows;
  const int64_t an = arow ? arho / d : 0;
  const int am = arow ? static_cast<int>(arho - an * d) : 0;
  const float* __restrict__ abase = MODE == kForward   ? in + an * a.xwidth + g.xoff + static_cast<int64_t>(am) * C
                                    : MODE == kInputGrad ? in + an * a.ywidth + g.yoff + am
                                                         : in + an * a.xwidth + g.xoff + am;
  // !FWD B staging: thread t holds weight row k0 + t / 8, columns c0 + CPT (t % 8) .. + CPT - 1
  // (CPT = TN / 8: two or four float4 loads), stored transposed element by element.  The k index
  // of B column col is XOR-swizzled by bsw(col) (a multiple of 8 below 32, so every aligned
  // 4-group of k stays contiguous and in its row; it follows col / 8 for CPT 8, col / 16 for
  // CPT 16, the bits that tell the lanes of one store apart): the transposed stores of a wave
  // then meet at most two lanes per bank, and with the 36-float pitch the 16-byte MFMA operand
  // reads stay conflict-free.
  constexpr int CPT = TN / 8;
  const int wk = tid >> 3, wc = (tid & 7) * CPT;
  auto bsw = [](int col) { return FWD ? 0 : ((col >> (CPT == 16 ? 4 : 3)) & 3) * 8; };
  f32x4_t acc[NT] = {};
  const int fr = lane & 15, fq = (lane >> 4) * 4;
  auto mfma_chunk = [&](int buf) {
#pragma unroll
    for (int kg = 0; kg < kKc; kg += 16) {
      const f32x4_t av = *reinterpret_cast<const f32x4_t*>(&sA[buf][wave * 16 + fr][kg + fq]);
      if constexpr (NBUF == 1) {
        // one B operand live at a time (the register budget of 8 waves per SIMD); the
        // accumulation chains of the other resident waves fill the MFMA pipe
#pragma unroll
        for (int t = 0; t < NT; t += 2) {
          const f32x4_t bv0 = *reinterpret_cast<const f32x4_t*>(&sB[buf][t * 16 + fr][(kg + fq) ^ bsw(t * 16 + fr)]);
          const f32x4_t bv1 = *reinterpret_cast<const f32x4_t*>(&sB[buf][t * 16 + 16 + fr][(kg + fq) ^ bsw(t * 16 + 16 + fr)]);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j], bv0[j], acc[t], 0, 0, 0);
            acc[t + 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j], bv1[j], acc[t + 1], 0, 0, 0);
          }
        }
      } else {
        f32x4_t bv[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t)
          bv[t] = *reinterpret_cast<const f32x4_t*>(&sB[buf][t * 16 + fr][(kg + fq) ^ bsw(t * 16 + fr)]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
          for (int t = 0; t < NT; ++t) acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j], bv[t][j], acc[t], 0, 0, 0);
        }
      }
    }
  };
  if constexpr (VEC) {
    // registers of one chunk: A (8 floats of the thread's row), B (8 floats, or CPT of the
    // input adjoint's weight row)
    constexpr int NRB = FWD ? 2 : CPT / 4;
    f32x4_t ra0, ra1, rb[NRB];
    // Every K chunk is full under VEC (kdim a multiple of 32), and no load is conditional on the
    // lane: a select or a branch on a loaded value would wait for the load at the fetch instead of
    // at the stage.  Rows past the end read row 0 and columns past the end read the last valid
    // weight columns: their products land in output rows / columns that are never stored.
    auto fetch = [&](int k0) {
      if constexpr (STRIDED) {   // mul_ir row: stride d over K
        const float* p = abase + (k0 + akq) * d;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          ra0[u] = p[u * d];
          ra1[u] = p[(u + 4) * d];
        }
      } else {
        const int blk = k0 / C, c = k0 - blk * C + akq;
        const float* p = abase + blk * d * C + c;
        ra0 = *reinterpret_cast<const f32x4_t*>(p);
        ra1 = *reinterpret_cast<const f32x4_t*>(p + 4);
      }
      if constexpr (FWD) {
        const int col = c0 + ar < ncols ? c0 + ar : ncols - 1;   // weight row col, 8 consecutive k
        const float* p = g.w + static_cast<int64_t>(col) * g.k + k0 + akq;
        rb[0] = *reinterpret_cast<const f32x4_t*>(p);
        rb[1] = *reinterpret_cast<const f32x4_t*>(p + 4);
      } else {
        // ncols (counts C) is a multiple of 32 and CPT is 8 or 16: the clamped run of CPT
        // columns stays in range
        const int col = c0 + wc < ncols ? c0 + wc : ncols - CPT;
        const float* p = g.w + static_cast<int64_t>(k0 + wk) * g.k + col;
#pragma unroll
        for (int q = 0; q < NRB; ++q) rb[q] = *reinterpret_cast<const f32x4_t*>(p + 4 * q);
      }
    };
    auto stage = [&](int buf) {
      *reinterpret_cast<f32x4_t*>(&sA[buf][ar][akq]) = ra0;
      *reinterpret_cast<f32x4_t*>(&sA[buf][ar][akq + 4]) = ra1;
      if constexpr (FWD) {
        *reinterpret_cast<f32x4_t*>(&sB[buf][ar][akq]) = rb[0];
        *reinterpret_cast<f32x4_t*>(&sB[buf][ar][akq + 4]) = rb[1];
      } else {
#pragma unroll
        for (int q = 0; q < NRB; ++q)
#pragma unroll
          for (int u = 0; u < 4; ++u) sB[buf][wc + 4 * q + u][wk ^ bsw(wc + 4 * q + u)] = rb[q][u];
      }
    };
    if (kdim > 0) {   // uniform
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
  // the lane's four output rows rho0 .. rho0 + 3: one division, then (n, m) stepped
  const int64_t rho0 = r0 + wave * 16 + 4 * (lane >> 4);
  int64_t n = rho0 / d;
  int m = static_cast<int>(rho0 - n * d);
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    if (v > 0 && ++m == d) {
      m = 0;
      ++n;
    }
    if (rho0 + v >= g.rows) continue;
    float* __restrict__ orow = FWD ? out + n * a.ywidth + g.yoff + m : out + n * a.xwidth + g.xoff + m * C;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int col = c0 + t * 16 + (lane & 15);
      if (col >= ncols) continue;
      const float val = a.alpha * acc[t][v];
      if (FWD) {
        orow[col * d] = val;
      } else {
        const int blk = col / C, c = col - blk * C;
        orow[blk * d * C + c] = val;
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
  // two LDS buffers for the long K of the forward (counts C), one for the short K of the others;
  // the input adjoint's vector path takes 128 columns per block (its B tile is read once per
  // 64 x 128 outputs instead of 64 x 64)
  const bool vec = desc->channels % 32 == 0 && (MODE != kInputGrad || desc->out_channels % 32 == 0);
  constexpr int kTn = MODE == kInputGrad ? kTileIg : kTile;
  const int tn = vec ? kTn : kTile;
  const dim3 grid(static_cast<unsigned>(row_tiles), static_cast<unsigned>((max_cols + tn - 1) / tn),
                  static_cast<unsigned>(degrees));
  if (vec)
    hipLaunchKernelGGL((degree_linear_kernel<MODE, true, MODE == kForward ? 2 : 1, kTn>), grid, dim3(256), 0, stream,
                       in, out, a);
  else
    hipLaunchKernelGGL((degree_linear_kernel<MODE, false, 1, kTile>), grid, dim3(256), 0, stream, in, out, a);
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
