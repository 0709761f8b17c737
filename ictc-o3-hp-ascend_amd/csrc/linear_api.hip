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

#include "ictc_common.hpp"
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
// D -> y (mul_ir).  kMulIrT: kMulIr with the weights given transposed (B = W [K, O] rows read
// like kInputGrad's, so no transposed copy of W is made).  VEC (channels, and for kInputGrad and
// kMulIrT out_channels, multiples of 32): every
// 32-wide K chunk is full, each K chunk of an x row lies in one path block and weight rows are
// float4-aligned, so operands are fetched into registers one chunk ahead (their loads in flight
// while the MFMAs of the current chunk run); with two LDS buffers
// (NBUF 2) the next chunk is staged into the other buffer right after those MFMAs (one barrier per
// chunk), with one (NBUF 1, half the LDS and so twice the resident blocks) after a second barrier.
// The forward's long K (counts C) takes two buffers, the input adjoint's short K (O) one.
// Without VEC, element by element, one chunk at a time.
enum LinearMode { kForward = 0, kInputGrad = 1, kMulIr = 2, kMulIrT = 3 };

template <int MODE, bool VEC, int NBUF, int TN>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NBUF == 1 ? (TN > kTile ? 5 : 8) : 4)))
degree_linear_kernel(const float* __restrict__ in, float* __restrict__ out, const LinearArgs a) {
  constexpr bool FWD = MODE != kInputGrad;      // D -> mul_ir y rows
  constexpr bool BT = MODE == kInputGrad || MODE == kMulIrT;   // B = W rows over K (staged transposed)
  constexpr int NT = TN / 16;                   // 16-column MFMA tiles per wave
  static_assert(BT ? (TN == kTile || TN == kTileIg) : TN == kTile, "column tile");
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
  auto bsw = [](int col) { return BT ? ((col >> (CPT == 16 ? 4 : 3)) & 3) * 8 : 0; };
  const int wld = MODE == kInputGrad ? g.k : ncols;   // BT: floats per weight row (over the columns)
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
    constexpr int NRB = BT ? CPT / 4 : 2;
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
      if constexpr (!BT) {
        const int col = c0 + ar < ncols ? c0 + ar : ncols - 1;   // weight row col, 8 consecutive k
        const float* p = g.w + static_cast<int64_t>(col) * g.k + k0 + akq;
        rb[0] = *reinterpret_cast<const f32x4_t*>(p);
        rb[1] = *reinterpret_cast<const f32x4_t*>(p + 4);
      } else {
        // ncols is a multiple of 32 under VEC and CPT is 8 or 16: the clamped run of CPT
        // columns stays in range
        const int col = c0 + wc < ncols ? c0 + wc : ncols - CPT;
        const float* p = g.w + static_cast<int64_t>(k0 + wk) * wld + col;
#pragma unroll
        for (int q = 0; q < NRB; ++q) rb[q] = *reinterpret_cast<const f32x4_t*>(p + 4 * q);
      }
    };
    auto stage = [&](int buf) {
      *reinterpret_cast<f32x4_t*>(&sA[buf][ar][akq]) = ra0;
      *reinterpret_cast<f32x4_t*>(&sA[buf][ar][akq + 4]) = ra1;
      if constexpr (!BT) {
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
      if constexpr (!BT) {
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
              (kk < kdim && col < ncols) ? g.w[static_cast<int64_t>(kk) * wld + col] : 0.f;
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
  if (MODE == kMulIr || MODE == kMulIrT) {   // one channel block per degree: x mul_ir [N, C (L+1)^2]
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
  const bool vec = desc->channels % 32 == 0 &&
                   ((MODE != kInputGrad && MODE != kMulIrT) || desc->out_channels % 32 == 0);
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

// Weight adjoint per degree (the dense product the layouts above otherwise need rearranged
// copies for):  gW_l[o, j] = alpha * sum_{rows rho = n d + m} gy[n, o, m] * x[rho, j], with the x
// rows of the forward (kWgIrMul: x[n, k, m, c], j = k C + c) or of the mul_ir map (kWgMulIr:
// x[n, c, m] at offset C l^2, j = c).  The rows of a degree are split into ranges (range_rows, a
// multiple of the 32-row chunk sized so that every block of the launch is resident at once: the
// LDS of three blocks fits a CU, and a second partial round of blocks would idle most CUs); a
// block of kWgWaves waves computes the 128 (o) x 64 (j) partial of one range (each wave 128 /
// kWgWaves o x 64 j, v_mfma_f32_16x16x4_f32 over 32-row chunks staged through LDS, the next
// chunk's loads in flight
// during the current chunk's MFMAs) and stores it into the workspace; a second kernel sums the
// ranges in order and scales by alpha (fixed order: bit-identical run to run).  Rows past the end
// read zeros from the buffer range check (their offsets lie past the tensors).
enum WgLayout { kWgIrMul = 0, kWgMulIr = 1 };
constexpr int kWgMinRows = 256;   // shortest range (8 chunks)
constexpr int kWgBlocksPerCu = 3;  // 51,200 B of LDS per block
constexpr int kWgO = 128, kWgJ = 64;
constexpr int kWgWaves = 8;   // waves per block: 16 o rows x 64 j each
constexpr int kWgPitchA = kWgO + 4, kWgPitchB = kWgJ + 4;

struct WgDegree {
  int64_t rows;     // N d
  int d, k;         // 2l + 1, output columns (counts[l] C)
  int64_t xoff, yoff;
  int ranges, otiles, jtiles;
  int64_t tile0;    // first block of the degree
  int64_t ws0;      // first workspace float of the degree: [ranges][O][k]
  float* gw;        // [O, k] or null (not asked for)
};

struct WgArgs {
  WgDegree g[ICTC_LINEAR_MAX_DEGREES];
  int degrees;
  int64_t tiles;
  int64_t xwidth, ywidth;
  int C, O;
  int range_rows;
  float alpha;
  uint32_t xbytes, ybytes;
};

template <int LAYOUT>
__global__ void __launch_bounds__(64 * kWgWaves)
degree_linear_wgrad_kernel(const float* __restrict__ gy, const float* __restrict__ x, float* __restrict__ ws,
                           const WgArgs a) {
  // XCD-contiguous block order: the column tiles of one row range (which read the same gY rows)
  // run on one XCD and share its L2
  const int64_t b = xcd_block(blockIdx.x, gridDim.x);
  int z = 0;
  while (z + 1 < a.degrees && b >= a.g[z + 1].tile0) ++z;
  const WgDegree g = a.g[z];
  if (g.gw == nullptr) return;   // uniform: the degree's gradient is not asked for
  const int64_t t = b - g.tile0;
  const int ot = static_cast<int>(t % g.otiles);
  const int64_t rest = t / g.otiles;
  const int jt = static_cast<int>(rest % g.jtiles);
  const int range = static_cast<int>(rest / g.jtiles);
  const int o0 = ot * kWgO, j0 = jt * kWgJ;
  const int64_t r0 = static_cast<int64_t>(range) * a.range_rows;
  const int64_t r1 = r0 + a.range_rows < g.rows ? r0 + a.range_rows : g.rows;
  const int d = g.d, C = a.C, O = a.O;
  __shared__ float sA[2][32][kWgPitchA];   // [buffer][row][o]
  __shared__ float sB[2][32][kWgPitchB];   // [buffer][row][j]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const rsrc_t ry = make_rsrc(gy, a.ybytes), rx = make_rsrc(x, a.xbytes);
  // A staging: element e = tid + T i (T threads, i < NA): o = e % 128, row e / 128; o past O (or
  // past the tile) reads o = 0 of its row: those accumulator rows are never stored.
  constexpr int T = 64 * kWgWaves, NA = 32 * kWgO / T, NB = 32 * kWgJ / T, AR = T / kWgO, BR = T / kWgJ;
  constexpr int OU = kWgO / 16 / kWgWaves;   // 16-row MFMA tiles per wave
  const int ao = tid & 127, arr = tid >> 7;
  const int aoc = o0 + ao < O ? o0 + ao : 0;
  // B staging: element e = tid + T i (i < NB): j = e % 64, row e / 64; j past k reads column 0
  const int bj = tid & 63, brr = tid >> 6;
  const int bjc = j0 + bj < g.k ? j0 + bj : 0;
  uint32_t bcol;   // byte offset of column bjc inside a row's degree block (m = 0)
  if constexpr (LAYOUT == kWgIrMul) {
    const int blk = bjc / C, c = bjc - blk * C;
    bcol = static_cast<uint32_t>(blk * d * C + c) * 4u;
  } else {
    bcol = static_cast<uint32_t>(bjc * d) * 4u;
  }
  // Row rho = n d + m of a chunk starting at c0 = n0 d + m0: the row q of the chunk has
  // n = n0 + (m0 + q) / d, computed as floor((m0 + q + 0.5) / d) in float (exact: m0 + q < 47 and
  // the rounding error is far below 0.5 / d).  Offsets are 32-bit bytes (tensors below 2 GiB).
  const float inv_d = 1.f / static_cast<float>(d);
  const uint32_t yw4 = static_cast<uint32_t>(a.ywidth) * 4u, xw4 = static_cast<uint32_t>(a.xwidth) * 4u;
  const uint32_t yo4 = static_cast<uint32_t>(g.yoff) * 4u + static_cast<uint32_t>(aoc * d) * 4u;
  const uint32_t xo4 = static_cast<uint32_t>(g.xoff) * 4u + bcol;
  const uint32_t mstep = (LAYOUT == kWgIrMul ? static_cast<uint32_t>(C) : 1u) * 4u;
  float ra[NA], rb[NB];
  auto fetch = [&](int64_t c0) {
    const int n0 = static_cast<int>(c0 / d), m0 = static_cast<int>(c0 - static_cast<int64_t>(n0) * d);
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int q = m0 + arr + AR * i;
      const int dn = static_cast<int>((static_cast<float>(q) + 0.5f) * inv_d), m = q - dn * d;
      // rows past r1 belong to the next range (or past the end): an out-of-range offset reads 0
      const uint32_t off = c0 + arr + AR * i < r1 ? static_cast<uint32_t>(n0 + dn) * yw4 + yo4 + static_cast<uint32_t>(m) * 4u
                                                  : 0xFFFFFFF0u;
      ra[i] = buf_load<1>(ry, off).v[0];
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int q = m0 + brr + BR * i;
      const int dn = static_cast<int>((static_cast<float>(q) + 0.5f) * inv_d), m = q - dn * d;
      const uint32_t off = c0 + brr + BR * i < r1 ? static_cast<uint32_t>(n0 + dn) * xw4 + xo4 + static_cast<uint32_t>(m) * mstep
                                                  : 0xFFFFFFF0u;
      rb[i] = buf_load<1>(rx, off).v[0];
    }
  };
  auto stage = [&](int buf) {
#pragma unroll
    for (int i = 0; i < NA; ++i) sA[buf][arr + AR * i][ao] = ra[i];
#pragma unroll
    for (int i = 0; i < NB; ++i) sB[buf][brr + BR * i][bj] = rb[i];
  };
  f32x4_t acc[OU][4] = {};
  const int fr = lane & 15, fq = (lane >> 4) * 4;
  auto mfma_chunk = [&](int buf) {
#pragma unroll
    for (int kg = 0; kg < 32; kg += 16) {
      float av[OU][4], bv[4][4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int u = 0; u < OU; ++u) av[u][j] = sA[buf][kg + fq + j][wave * 16 * OU + u * 16 + fr];
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) bv[tt][j] = sB[buf][kg + fq + j][tt * 16 + fr];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int u = 0; u < OU; ++u)
#pragma unroll
          for (int tt = 0; tt < 4; ++tt)
            acc[u][tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u][j], bv[tt][j], acc[u][tt], 0, 0, 0);
    }
  };
  fetch(r0);
  stage(0);
  __syncthreads();
  int buf = 0;
  for (int64_t c0 = r0; c0 < r1; c0 += 32) {
    const bool more = c0 + 32 < r1;
    if (more) fetch(c0 + 32);
    mfma_chunk(buf);
    if (more) stage(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }
  float* __restrict__ part = ws + g.ws0 + static_cast<int64_t>(range) * O * g.k;
#pragma unroll
  for (int u = 0; u < OU; ++u)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int o = o0 + wave * 16 * OU + u * 16 + 4 * (lane >> 4) + v;
      if (o >= O) continue;
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const int j = j0 + tt * 16 + fr;
        if (j < g.k) part[static_cast<int64_t>(o) * g.k + j] = acc[u][tt][v];
      }
    }
}

// gW_l = alpha * the sum of the degree's range partials, in range order (one thread per entry).
__global__ void __launch_bounds__(256) degree_linear_wgrad_sum_kernel(const float* __restrict__ ws, const WgArgs a,
                                                                      int64_t entries) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < entries;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    int64_t base = 0;
    int z = 0;
    for (; z < a.degrees; ++z) {
      const int64_t n = static_cast<int64_t>(a.O) * a.g[z].k;
      if (i < base + n) break;
      base += n;
    }
    const WgDegree& g = a.g[z];
    if (g.gw == nullptr) continue;
    const int64_t e = i - base, stride = static_cast<int64_t>(a.O) * g.k;
    const float* p = ws + g.ws0 + e;
    float s = 0.f;
    int r = 0;
    for (; r + 4 <= g.ranges; r += 4) {   // four loads in flight, added in range order
      const float v0 = p[r * stride], v1 = p[(r + 1) * stride], v2 = p[(r + 2) * stride], v3 = p[(r + 3) * stride];
      s = (((s + v0) + v1) + v2) + v3;
    }
    for (; r < g.ranges; ++r) s += p[r * stride];
    g.gw[e] = a.alpha * s;
  }
}

// Workspace floats of one weight-adjoint call, and the launch geometry (0 for an empty call).
int wgrad_prepare(const ictc_degree_linear_desc* desc, int layout, float alpha, int64_t nodes, float* const* grad_w,
                  WgArgs* a, int64_t* ws_floats, int64_t* entries) {
  if (desc == nullptr || nodes < 0 || (layout != kWgIrMul && layout != kWgMulIr)) return ICTC_ERR_INVALID_ARGUMENT;
  if (desc->lmax < 0 || desc->lmax >= ICTC_LINEAR_MAX_DEGREES || desc->channels < 1 || desc->out_channels < 1)
    return ICTC_ERR_INVALID_ARGUMENT;
  *a = WgArgs{};
  a->degrees = desc->lmax + 1;
  a->C = desc->channels;
  a->O = desc->out_channels;
  a->alpha = alpha;
  int64_t xw = 0;
  for (int l = 0; l <= desc->lmax; ++l) {
    if (desc->counts[l] < 0) return ICTC_ERR_INVALID_ARGUMENT;
    if (layout == kWgMulIr && desc->counts[l] != 1) return ICTC_ERR_INVALID_ARGUMENT;
    xw += static_cast<int64_t>(desc->counts[l]) * (2 * l + 1) * desc->channels;
  }
  a->xwidth = xw;
  a->ywidth = static_cast<int64_t>(desc->out_channels) * (desc->lmax + 1) * (desc->lmax + 1);
  const int64_t xb = nodes * a->xwidth * 4, yb = nodes * a->ywidth * 4;
  if (xb >= 0x7FFFFFF0 || yb >= 0x7FFFFFF0) return ICTC_ERR_UNSUPPORTED;   // 32-bit buffer offsets
  a->xbytes = static_cast<uint32_t>(xb);
  a->ybytes = static_cast<uint32_t>(yb);
  int64_t xoff = 0, work = 0, columns = 0;
  for (int l = 0; l <= desc->lmax; ++l) {
    WgDegree& g = a->g[l];
    g.d = 2 * l + 1;
    g.rows = nodes * g.d;
    g.k = desc->counts[l] * desc->channels;
    g.xoff = layout == kWgIrMul ? xoff : static_cast<int64_t>(desc->channels) * l * l;
    g.yoff = static_cast<int64_t>(desc->out_channels) * l * l;
    g.gw = g.k > 0 ? grad_w[l] : nullptr;
    xoff += static_cast<int64_t>(g.k) * g.d;
    g.otiles = (desc->out_channels + kWgO - 1) / kWgO;
    g.jtiles = (g.k + kWgJ - 1) / kWgJ;
    if (g.gw) {
      work += g.rows * g.otiles * g.jtiles;
      columns += static_cast<int64_t>(g.otiles) * g.jtiles;
    }
  }
  // ranges: blocks = sum ceil(rows / R) tiles <= work / R + columns <= the resident capacity
  const int64_t room = static_cast<int64_t>(kWgBlocksPerCu) * compute_units() - columns;
  int64_t rr = room > 0 ? (work + room - 1) / room : work;
  rr = (rr + 31) / 32 * 32;
  a->range_rows = static_cast<int>(rr < kWgMinRows ? kWgMinRows : (rr > (1 << 30) ? (1 << 30) : rr));
  int64_t tiles = 0, ws = 0, ent = 0;
  for (int l = 0; l <= desc->lmax; ++l) {
    WgDegree& g = a->g[l];
    g.ranges = g.gw ? static_cast<int>((g.rows + a->range_rows - 1) / a->range_rows) : 0;
    g.tile0 = tiles;
    g.ws0 = ws;
    tiles += static_cast<int64_t>(g.ranges) * g.otiles * g.jtiles;
    ws += static_cast<int64_t>(g.ranges) * desc->out_channels * g.k;
    ent += static_cast<int64_t>(desc->out_channels) * g.k;
  }
  a->tiles = tiles;
  *ws_floats = ws;
  *entries = ent;
  return ICTC_OK;
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

int ictc_hip_degree_linear_mul_ir_transposed(const ictc_degree_linear_desc* desc, const float* x,
                                             const float* const* weights, float alpha, float* y, int64_t nodes,
                                             hipStream_t stream) {
  return ictc::launch<ictc::kMulIrT>(desc, x, weights, alpha, y, nodes, stream);
}

int64_t ictc_hip_degree_linear_weight_grad_workspace(const ictc_degree_linear_desc* desc, int x_layout,
                                                     int64_t nodes) {
  float* none[ICTC_LINEAR_MAX_DEGREES];
  float dummy = 0.f;
  for (int l = 0; l < ICTC_LINEAR_MAX_DEGREES; ++l) none[l] = &dummy;   // every degree asked for
  ictc::WgArgs a;
  int64_t ws = 0, entries = 0;
  const int st = ictc::wgrad_prepare(desc, x_layout, 1.f, nodes, none, &a, &ws, &entries);
  return st == ICTC_OK ? ws : -static_cast<int64_t>(st);
}

int ictc_hip_degree_linear_weight_grad(const ictc_degree_linear_desc* desc, int x_layout, const float* grad_y,
                                       const float* x, float alpha, float* workspace, int64_t workspace_floats,
                                       float* const* grad_weights, int64_t nodes, hipStream_t stream) {
  if (grad_weights == nullptr) return ICTC_ERR_INVALID_ARGUMENT;
  ictc::WgArgs a;
  int64_t ws = 0, entries = 0;
  const int st = ictc::wgrad_prepare(desc, x_layout, alpha, nodes, grad_weights, &a, &ws, &entries);
  if (st != ICTC_OK) return st;
  if (entries == 0) return ICTC_OK;
  // no rows: no ranges, and the sum kernel writes zero gradients
  if (nodes > 0 && (grad_y == nullptr || x == nullptr || workspace == nullptr || workspace_floats < ws))
    return ICTC_ERR_INVALID_ARGUMENT;
  if (a.tiles > 0x7fffffff) return ICTC_ERR_UNSUPPORTED;
  if (a.tiles > 0) {
    if (x_layout == ictc::kWgIrMul)
      hipLaunchKernelGGL(ictc::degree_linear_wgrad_kernel<ictc::kWgIrMul>, dim3(static_cast<unsigned>(a.tiles)),
                         dim3(64 * ictc::kWgWaves), 0, stream, grad_y, x, workspace, a);
    else
      hipLaunchKernelGGL(ictc::degree_linear_wgrad_kernel<ictc::kWgMulIr>, dim3(static_cast<unsigned>(a.tiles)),
                         dim3(64 * ictc::kWgWaves), 0, stream, grad_y, x, workspace, a);
    if (hipGetLastError() != hipSuccess) return ICTC_ERR_LAUNCH;
  }
  const int64_t blocks = (entries + 255) / 256;
  hipLaunchKernelGGL(ictc::degree_linear_wgrad_sum_kernel, dim3(static_cast<unsigned>(blocks < 4096 ? blocks : 4096)),
                     dim3(256), 0, stream, workspace, a, entries);
  return hipGetLastError() == hipSuccess ? ICTC_OK : ICTC_ERR_LAUNCH;
}

}  // extern "C"
