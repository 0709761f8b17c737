// Radial MLP of the MACE interaction on the matrix cores (gfx950, v_mfma_f32_16x16x4_f32).
//
// The interaction's radial network up to its last Linear (reference
// mace_ictc/models/pure_cartesian_ictd_fix.py:1545-1553, applied at :1795; the normalised SiLU
// of :610-619), per edge:
//   z1 = W1 f,  a1 = silu(z1),  z2 = s W2 a1,  a2 = silu(z2),  z3 = s W3 a2,  h = silu(z3)
// with f [E, B] (B <= 16 basis functions), W1 [64, B], W2, W3 [64, 64] (nn.Linear [out, in]) and s
// the normalised-SiLU constant folded into the layer that follows it.  Modes:
//   VALUE   : h                                                        [E, 64]
//   VJP     : for an adjoint g of h: J^T g (feature gradient, [E, B]) and the weight gradients
//   VJP_VJP : for g and a cotangent u of that feature gradient, the derivatives of <u, J^T g>:
//             J u (its gradient in g, [E, 64]), its gradients in f and in the three weights
//             (force training's double backward)
// where a composition of library ops runs one GEMM per layer and direction plus several
// elementwise passes per activation (some forty launches per interaction in force training).
// With sg = sigmoid(z): silu' = sg (1 + z (1 - sg)), silu'' = sg (1 - sg) (2 + z (1 - 2 sg)).
// VJP_VJP, with the tangent t1 = W1 u, ta1 = silu'(z1) t1, t2 = s W2 ta1, ta2 = silu'(z2) t2,
// t3 = s W3 ta2, runs the reverse sweep of <g, silu'(z3) t3> over both the tangent and the primal:
//   A3 = g silu'(z3),  B3 = g t3 silu''(z3)
//   A2 = silu'(z2) s W3^T A3,  B2 = (s W3^T A3) t2 silu''(z2) + silu'(z2) s W3^T B3     (same for 1)
//   dW3 = s (A3 ta2^T + B3 a2^T), dW2 = s (A2 ta1^T + B2 a1^T), dW1 = A1 u^T + B1 f^T,  df = W1^T B1
// summed over edges.
//
// Layout.  A wave owns 16 edges at a time.  Every product is computed transposed,
// out^T [64 x 16 edges] = W [64 x K] act^T [K x 16 edges], as 16 x 16 MFMA tiles: the result sits in
// the accumulator layout (lane l: edge l % 16, features 16 t + 4 (l / 16) + v, v = 0..3, tile t),
// and that layout is directly the B operand of the next product when its four consecutive MFMAs
// take the reduction index 16 g + 4 (l / 16) + j (j = 0..3): activations stay in registers from
// layer to layer.  The weights (s folded in) sit in LDS; a forward product reads its A operand as
// one 16-byte row slice per four MFMAs, an adjoint product (W^T c) single floats down a column.
// Weight gradients reduce over edges, which the MFMA takes from the lane-group index: the wave
// stages its two [64 x 16] factors feature-major in LDS, reads them back as 16-byte edge slices and
// accumulates the 64 x 64 products in registers over all of its tiles.  The four waves of a block
// then add theirs in LDS in wave order, the block writes one partial, and a second kernel sums the
// partials in block order: the gradients are bit-identical from run to run.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "ictc_common.hpp"

namespace ictc {
namespace {

constexpr int kRw = ICTC_RADIAL_WIDTH;   // 64
constexpr int kRb = ICTC_RADIAL_MAX_BASIS;  // 16
constexpr int kRWaves = 4;
constexpr int kRThreads = kWave * kRWaves;
constexpr int kLdW = kRw + 4;            // LDS row stride of W2, W3 (floats)
constexpr int kLdW1 = kRb + 4;           // of W1 (zero-padded to 16 inputs)
constexpr int kLdS = 4 * 16 + 4;         // of a staged [feature][64 edges] factor
constexpr int kStage = 2 * kRw * kLdS;   // floats of the block's staging area (two factors)
constexpr int kPart = kRw * kRb + 2 * kRw * kRw;   // one block's partial: dW1 [64][16], dW2, dW3
// Weight-gradient launches: blocks per CU (the VJP kernel's registers allow two resident blocks,
// the double backward's one); the workspace is sized for the larger count.
constexpr int kRBlocksPerCuVjp = 2;
constexpr int kRBlocksPerCuVjpVjp = 1;
constexpr int kSumRows = 16;             // partial entries per block of the sum kernel ...
constexpr int kSumParts = 16;            // ... each summed by this many threads

static_assert(kRw == 64 && kRb == 16, "tiling assumes 64 hidden features and at most 16 basis functions");
static_assert(kSumRows * kSumParts == 256 && kPart % kSumRows == 0, "sum kernel geometry");

struct RadialArgs {
  const float* f;    // [E, B]
  const float* w1;   // [64, B]
  const float* w2;   // [64, 64]
  const float* w3;   // [64, 64]
  const float* g;    // [E, 64] adjoint of h (VJP, VJP_VJP)
  const float* u;    // [E, B]  cotangent of the feature gradient (VJP_VJP)
  float* h;          // [E, 64] VALUE
  float* gf;         // [E, B]  VJP: J^T g; VJP_VJP: gradient in f (optional)
  float* gg;         // [E, 64] VJP_VJP: J u (optional)
  float* ws;         // [blocks, kPart] weight-gradient partials (optional)
  int64_t edges;
  int64_t tiles;     // ceil(E / 16)
  int basis;
  float scale;
};

// 64 features x 16 edges in the accumulator layout.
struct T64 {
  f32x4 t[4];
};

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

__device__ __forceinline__ f32x4 mfma(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// out = W x: W [64][kLdW] in LDS, x in the accumulator layout.
__device__ __forceinline__ T64 forward64(const float* W, const T64& x, int r, int q) {
  T64 z;
#pragma unroll
  for (int o = 0; o < 4; ++o) z.t[o] = zero4();
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    f32x4 w[4];
#pragma unroll
    for (int o = 0; o < 4; ++o) w[o] = *reinterpret_cast<const f32x4*>(W + (16 * o + r) * kLdW + 16 * g + 4 * q);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int o = 0; o < 4; ++o) z.t[o] = mfma(w[o][j], x.t[g][j], z.t[o]);
  }
  return z;
}

// out = W1 x0, x0 = the lane's basis values 4 q + j (j = 0..3) of edge r (zero past B).
__device__ __forceinline__ T64 forward_first(const float* W1, f32x4 x0, int r, int q) {
  T64 z;
  f32x4 w[4];
#pragma unroll
  for (int o = 0; o < 4; ++o) {
    z.t[o] = zero4();
    w[o] = *reinterpret_cast<const f32x4*>(W1 + (16 * o + r) * kLdW1 + 4 * q);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int o = 0; o < 4; ++o) z.t[o] = mfma(w[o][j], x0[j], z.t[o]);
  return z;
}

// out = W^T c: c over W's 64 outputs, out over its 64 inputs (accumulator layout).
__device__ __forceinline__ T64 adjoint64(const float* W, const T64& c, int r, int q) {
  T64 y;
#pragma unroll
  for (int k = 0; k < 4; ++k) y.t[k] = zero4();
#pragma unroll
  for (int g = 0; g < 4; ++g)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float* col = W + (16 * g + 4 * q + j) * kLdW + r;
      float a[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) a[k] = col[16 * k];
#pragma unroll
      for (int k = 0; k < 4; ++k) y.t[k] = mfma(a[k], c.t[g][j], y.t[k]);
    }
  return y;
}

// out = W1^T c: lane (r, q) receives the gradient of basis function 4 q + v of edge r.
__device__ __forceinline__ f32x4 adjoint_first(const float* W1, const T64& c, int r, int q) {
  f32x4 y = zero4();
#pragma unroll
  for (int g = 0; g < 4; ++g)
#pragma unroll
    for (int j = 0; j < 4; ++j) y = mfma(W1[(16 * g + 4 * q + j) * kLdW1 + r], c.t[g][j], y);
  return y;
}

__device__ __forceinline__ float sigmoid(float z) { return __builtin_amdgcn_rcpf(1.f + __expf(-z)); }

// Elementwise maps over a tile.
template <typename F>
__device__ __forceinline__ T64 map64(F&& fn) {
  T64 o;
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) o.t[t][v] = fn(t, v);
  return o;
}

__device__ __forceinline__ T64 sigmoid64(const T64& z) {
  return map64([&](int t, int v) { return sigmoid(z.t[t][v]); });
}
__device__ __forceinline__ T64 silu64(const T64& z, const T64& s) {
  return map64([&](int t, int v) { return z.t[t][v] * s.t[t][v]; });
}
// silu'(z) = s (1 + z (1 - s))
__device__ __forceinline__ float dsilu(float z, float s) { return s * fmaf(z, 1.f - s, 1.f); }
// silu''(z) = s (1 - s) (2 + z (1 - 2 s))
__device__ __forceinline__ float d2silu(float z, float s) { return s * (1.f - s) * fmaf(z, fmaf(-2.f, s, 1.f), 2.f); }

// g[row] in the accumulator layout (zero for a dead lane).
__device__ __forceinline__ T64 load64(const float* p, int64_t row, bool live, int q) {
  T64 x;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(p + row * kRw + 16 * t + 4 * q);
    x.t[t] = live ? v : zero4();
  }
  return x;
}

__device__ __forceinline__ void store64(float* p, int64_t row, bool live, int q, const T64& x) {
  if (!live) return;
#pragma unroll
  for (int t = 0; t < 4; ++t) *reinterpret_cast<f32x4*>(p + row * kRw + 16 * t + 4 * q) = x.t[t];
}

// The lane's basis values 4 q + j of a row (zero past B, and everywhere for a dead lane if asked).
__device__ __forceinline__ f32x4 load_basis(const float* p, int64_t row, int basis, int q, bool keep) {
  f32x4 x;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int k = 4 * q + j;
    x[j] = (keep && k < basis) ? p[row * basis + k] : 0.f;
  }
  return x;
}

// Weight gradients.  A round is four tiles, one per wave (64 edges).  For each factor pair the
// waves stage their tiles feature-major side by side, S[feature][16 w + edge], and after a block
// barrier wave w accumulates rows 16 w .. 16 w + 15 of the gradient over all 64 edges: its
// accumulators hold one 16-row band of each weight gradient (9 MFMA tiles).
struct WgradAcc {
  f32x4 w3[4], w2[4], w1;
};

__device__ __forceinline__ void stage64(float* S, const T64& x, int r, int q, int wave) {
#pragma unroll
  for (int g = 0; g < 4; ++g)
#pragma unroll
    for (int v = 0; v < 4; ++v) S[(16 * g + 4 * q + v) * kLdS + 16 * wave + r] = x.t[g][v];
}
__device__ __forceinline__ void stage16(float* S, f32x4 x, int r, int q, int wave) {
#pragma unroll
  for (int v = 0; v < 4; ++v) S[(4 * q + v) * kLdS + 16 * wave + r] = x[v];
}

// acc[k] (rows 16 w.., cols 16 k..) += sum over the round's 64 edges of X[e][row] Y[e][col].
template <int NK>
__device__ __forceinline__ void accumulate(f32x4* acc, const float* SX, const float* SY, int r, int q, int wave) {
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    const f32x4 av = *reinterpret_cast<const f32x4*>(SX + (16 * wave + r) * kLdS + 16 * kk + 4 * q);
    f32x4 bv[NK];
#pragma unroll
    for (int k = 0; k < NK; ++k) bv[k] = *reinterpret_cast<const f32x4*>(SY + (16 * k + r) * kLdS + 16 * kk + 4 * q);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int k = 0; k < NK; ++k) acc[k] = mfma(av[j], bv[k][j], acc[k]);
  }
}

// acc += X^T Y over the round (Y 64 wide).  Block-uniform: every wave calls it.
__device__ __forceinline__ void pair64(f32x4 (&acc)[4], float* S, const T64& x, const T64& y, int r, int q,
                                       int wave) {
  stage64(S, x, r, q, wave);
  stage64(S + kRw * kLdS, y, r, q, wave);
  __syncthreads();
  accumulate<4>(acc, S, S + kRw * kLdS, r, q, wave);
  __syncthreads();
}
// acc += X^T Y over the round (Y the 16 basis values).
__device__ __forceinline__ void pair16(f32x4& acc, float* S, const T64& x, f32x4 y, int r, int q, int wave) {
  stage64(S, x, r, q, wave);
  stage16(S + kRw * kLdS, y, r, q, wave);
  __syncthreads();
  accumulate<1>(&acc, S, S + kRw * kLdS, r, q, wave);
  __syncthreads();
}

// One layer's activation from its pre-activation z: a = silu(z) and d = silu'(z) (z itself is
// not kept).
struct Act {
  T64 a, d;
};

__device__ __forceinline__ Act activate(const T64& z) {
  Act o;
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float zv = z.t[t][v], sv = sigmoid(zv);
      o.a.t[t][v] = zv * sv;
      o.d.t[t][v] = dsilu(zv, sv);
    }
  return o;
}

__device__ __forceinline__ T64 mul64(const T64& x, const T64& y) {
  return map64([&](int t, int v) { return x.t[t][v] * y.t[t][v]; });
}
// silu'(z) x from (z, sigmoid(z))
__device__ __forceinline__ T64 dmul64(const T64& z, const T64& s, const T64& x) {
  return map64([&](int t, int v) { return dsilu(z.t[t][v], s.t[t][v]) * x.t[t][v]; });
}

// MODE: ICTC_RADIAL_*; WG: the launch accumulates weight gradients (persistent blocks, block
// barriers in the weight-gradient phases).
template <int MODE, bool WG>
__global__ void __launch_bounds__(kRThreads) radial_mlp_kernel(const RadialArgs a) {
  __shared__ __align__(16) float sW1[kRw * kLdW1];
  __shared__ __align__(16) float sW2[kRw * kLdW];
  __shared__ __align__(16) float sW3[kRw * kLdW];
  __shared__ __align__(16) float sS[WG ? kStage : 4];

  for (int i = threadIdx.x; i < kRw * kRb; i += kRThreads) {
    const int o = i / kRb, k = i % kRb;
    sW1[o * kLdW1 + k] = k < a.basis ? a.w1[o * a.basis + k] : 0.f;
  }
  for (int i = threadIdx.x; i < kRw * kRw; i += kRThreads) {
    const int o = i / kRw, k = i % kRw;
    sW2[o * kLdW + k] = a.scale * a.w2[i];
    sW3[o * kLdW + k] = a.scale * a.w3[i];
  }
  __syncthreads();

  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int r = lane & 15, q = lane >> 4;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * a.tiles / gridDim.x;
  const int64_t t1 = static_cast<int64_t>(blockIdx.x + 1) * a.tiles / gridDim.x;
  // with weight gradients every wave runs the same number of rounds (their phases hold block
  // barriers); a tile past the block's range is computed on dead lanes and contributes zero
  const int64_t rounds = (t1 - t0 + kRWaves - 1) / kRWaves;
  WgradAcc acc;
  if constexpr (WG) {
#pragma unroll
    for (int i = 0; i < 4; ++i) acc.w3[i] = acc.w2[i] = zero4();
    acc.w1 = zero4();
  }

  for (int64_t i = 0; i < rounds; ++i) {
    const int64_t t = t0 + kRWaves * i + wave;
    if (!WG && t >= t1) break;
    const int64_t e = t * 16 + r;
    const bool live = t < t1 && e < a.edges;
    const int64_t row = live ? e : a.edges - 1;
    const f32x4 x0 = load_basis(a.f, row, a.basis, q, true);
    if constexpr (MODE == ICTC_RADIAL_VALUE) {
      const T64 z1 = forward_first(sW1, x0, r, q);
      const T64 a1 = silu64(z1, sigmoid64(z1));
      const T64 z2 = forward64(sW2, a1, r, q);
      const T64 a2 = silu64(z2, sigmoid64(z2));
      const T64 z3 = forward64(sW3, a2, r, q);
      store64(a.h, row, live, q, silu64(z3, sigmoid64(z3)));
    } else if constexpr (MODE == ICTC_RADIAL_VJP) {
      const T64 g = load64(a.g, row, live, q);
      const Act L1 = activate(forward_first(sW1, x0, r, q));
      const Act L2 = activate(forward64(sW2, L1.a, r, q));
      const Act L3 = activate(forward64(sW3, L2.a, r, q));
      const T64 c3 = mul64(g, L3.d);
      if constexpr (WG) pair64(acc.w3, sS, c3, L2.a, r, q, wave);
      const T64 c2 = mul64(adjoint64(sW3, c3, r, q), L2.d);
      if constexpr (WG) pair64(acc.w2, sS, c2, L1.a, r, q, wave);
      const T64 c1 = mul64(adjoint64(sW2, c2, r, q), L1.d);
      if constexpr (WG) pair16(acc.w1, sS, c1, x0, r, q, wave);
      if (a.gf != nullptr) {   // the MFMA operands come from every lane: outside the live test
        const f32x4 d = adjoint_first(sW1, c1, r, q);
#pragma unroll
        for (int v = 0; v < 4; ++v)
          if (live && 4 * q + v < a.basis) a.gf[row * a.basis + 4 * q + v] = d[v];
      }
    } else {
      // (z, sigmoid(z)) per layer, from which silu, silu' and silu'' are rebuilt where used:
      // fewer live registers than keeping the three of them
      const f32x4 xu = load_basis(a.u, row, a.basis, q, live);
      const T64 z1 = forward_first(sW1, x0, r, q);
      const T64 s1 = sigmoid64(z1);
      const T64 t1v = forward_first(sW1, xu, r, q);
      const T64 z2 = forward64(sW2, silu64(z1, s1), r, q);
      const T64 s2 = sigmoid64(z2);
      const T64 t2v = forward64(sW2, dmul64(z1, s1, t1v), r, q);
      const T64 z3 = forward64(sW3, silu64(z2, s2), r, q);
      const T64 s3 = sigmoid64(z3);
      const T64 t3v = forward64(sW3, dmul64(z2, s2, t2v), r, q);
      const T64 g = load64(a.g, row, live, q);
      if (a.gg != nullptr) store64(a.gg, row, live, q, dmul64(z3, s3, t3v));
      const T64 A3 = dmul64(z3, s3, g);
      const T64 B3 = map64([&](int i, int v) { return g.t[i][v] * t3v.t[i][v] * d2silu(z3.t[i][v], s3.t[i][v]); });
      if constexpr (WG) {
        pair64(acc.w3, sS, A3, dmul64(z2, s2, t2v), r, q, wave);
        pair64(acc.w3, sS, B3, silu64(z2, s2), r, q, wave);
      }
      const T64 P2 = adjoint64(sW3, A3, r, q);
      const T64 Q2 = adjoint64(sW3, B3, r, q);
      const T64 A2 = dmul64(z2, s2, P2);
      const T64 B2 = map64([&](int i, int v) {
        return fmaf(P2.t[i][v] * t2v.t[i][v], d2silu(z2.t[i][v], s2.t[i][v]), Q2.t[i][v] * dsilu(z2.t[i][v], s2.t[i][v]));
      });
      if constexpr (WG) {
        pair64(acc.w2, sS, A2, dmul64(z1, s1, t1v), r, q, wave);
        pair64(acc.w2, sS, B2, silu64(z1, s1), r, q, wave);
      }
      const T64 P1 = adjoint64(sW2, A2, r, q);
      const T64 Q1 = adjoint64(sW2, B2, r, q);
      const T64 B1 = map64([&](int i, int v) {
        return fmaf(P1.t[i][v] * t1v.t[i][v], d2silu(z1.t[i][v], s1.t[i][v]), Q1.t[i][v] * dsilu(z1.t[i][v], s1.t[i][v]));
      });
      if constexpr (WG) {
        pair16(acc.w1, sS, dmul64(z1, s1, P1), xu, r, q, wave);
        pair16(acc.w1, sS, B1, x0, r, q, wave);
      }
      if (a.gf != nullptr) {
        const f32x4 d = adjoint_first(sW1, B1, r, q);
#pragma unroll
        for (int v = 0; v < 4; ++v)
          if (live && 4 * q + v < a.basis) a.gf[row * a.basis + 4 * q + v] = d[v];
      }
    }
  }

  if constexpr (WG) {   // the wave's row band of each gradient into the block's partial
    float* out = a.ws + static_cast<int64_t>(blockIdx.x) * kPart;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = 16 * wave + 4 * q + v;
      out[row * kRb + r] = acc.w1[v];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        out[kRw * kRb + row * kRw + 16 * k + r] = acc.w2[k][v];
        out[kRw * kRb + kRw * kRw + row * kRw + 16 * k + r] = acc.w3[k][v];
      }
    }
  }
}

// dW1 = sum of the dW1 partials, dW2 = s sum, dW3 = s sum (zero for no blocks).  Thread (c, p) of
// a block adds the partials of blocks p, p + kSumParts, ... for entry c with four loads in flight,
// and thread (c, 0) adds the kSumParts results in order: a fixed order, bit-identical run to run.
__global__ void __launch_bounds__(256) radial_wsum_kernel(const float* __restrict__ ws, int blocks, int basis,
                                                          float scale, float* __restrict__ gw1,
                                                          float* __restrict__ gw2, float* __restrict__ gw3) {
  __shared__ float part[kSumParts][kSumRows + 1];
  const int c = threadIdx.x % kSumRows, p = threadIdx.x / kSumRows;
  const int i = blockIdx.x * kSumRows + c;
  const float* src = ws + i;
  constexpr int kStep = kSumParts;
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
  int b = p;
  for (; b + 3 * kStep < blocks; b += 4 * kStep) {
    s0 += src[static_cast<int64_t>(b) * kPart];
    s1 += src[static_cast<int64_t>(b + kStep) * kPart];
    s2 += src[static_cast<int64_t>(b + 2 * kStep) * kPart];
    s3 += src[static_cast<int64_t>(b + 3 * kStep) * kPart];
  }
  for (; b < blocks; b += kStep) s0 += src[static_cast<int64_t>(b) * kPart];
  part[p][c] = (s0 + s1) + (s2 + s3);
  __syncthreads();
  if (p != 0) return;
  float tot = 0.f;
#pragma unroll
  for (int k = 0; k < kSumParts; ++k) tot += part[k][c];
  if (i < kRw * kRb) {
    const int o = i / kRb, k = i % kRb;
    if (gw1 != nullptr && k < basis) gw1[o * basis + k] = tot;
  } else if (i < kRw * kRb + kRw * kRw) {
    if (gw2 != nullptr) gw2[i - kRw * kRb] = scale * tot;
  } else if (gw3 != nullptr) {
    gw3[i - kRw * kRb - kRw * kRw] = scale * tot;
  }
}

int64_t radial_tiles(int64_t edges) { return (edges + 15) / 16; }

// Blocks of a weight-gradient launch (0 for no edges).
int radial_wgrad_blocks(int64_t edges, int mode) {
  const int64_t need = (radial_tiles(edges) + kRWaves - 1) / kRWaves;
  const int per_cu = mode == ICTC_RADIAL_VJP_VJP ? kRBlocksPerCuVjpVjp : kRBlocksPerCuVjp;
  const int64_t cap = static_cast<int64_t>(per_cu) * compute_units();
  return static_cast<int>(need < cap ? need : cap);
}

}  // namespace
}  // namespace ictc

extern "C" int64_t ictc_hip_radial_mlp_workspace(int64_t edges) {
  if (edges < 0) return -ICTC_ERR_INVALID_ARGUMENT;
  return static_cast<int64_t>(ictc::radial_wgrad_blocks(edges, ICTC_RADIAL_VJP)) * ictc::kPart;
}

extern "C" int ictc_hip_radial_mlp(int mode, const float* feats, const float* w1, const float* w2, const float* w3,
                                   float scale, const float* grad_hidden, const float* cotangent, float* out_hidden,
                                   float* out_grad_feats, float* out_grad_grad_hidden, float* workspace,
                                   int64_t workspace_floats, float* grad_w1, float* grad_w2, float* grad_w3,
                                   int num_basis, int64_t edges, hipStream_t stream) {
  using namespace ictc;
  if (mode < ICTC_RADIAL_VALUE || mode > ICTC_RADIAL_VJP_VJP) return ICTC_ERR_UNSUPPORTED;
  if (num_basis < 1 || num_basis > kRb) return ICTC_ERR_UNSUPPORTED;
  if (edges < 0 || w1 == nullptr || w2 == nullptr || w3 == nullptr) return ICTC_ERR_INVALID_ARGUMENT;
  const bool wgrad = mode != ICTC_RADIAL_VALUE && (grad_w1 != nullptr || grad_w2 != nullptr || grad_w3 != nullptr);
  if (mode == ICTC_RADIAL_VALUE) {
    if (edges > 0 && (out_hidden == nullptr || feats == nullptr)) return ICTC_ERR_INVALID_ARGUMENT;
  } else {
    const bool any = wgrad || out_grad_feats != nullptr ||
                     (mode == ICTC_RADIAL_VJP_VJP && out_grad_grad_hidden != nullptr);
    if (!any) return ICTC_OK;
    if (edges > 0 && (feats == nullptr || grad_hidden == nullptr)) return ICTC_ERR_INVALID_ARGUMENT;
    if (mode == ICTC_RADIAL_VJP_VJP && edges > 0 && cotangent == nullptr) return ICTC_ERR_INVALID_ARGUMENT;
  }
  const int64_t tiles = radial_tiles(edges);
  if (tiles > (static_cast<int64_t>(1) << 31) - 1) return ICTC_ERR_UNSUPPORTED;
  int blocks = 0;
  if (wgrad) {
    blocks = radial_wgrad_blocks(edges, mode);
    if (workspace == nullptr || workspace_floats < static_cast<int64_t>(blocks) * kPart)
      return ICTC_ERR_INVALID_ARGUMENT;
  }
  RadialArgs a{feats, w1, w2, w3, grad_hidden, cotangent, out_hidden, out_grad_feats,
               mode == ICTC_RADIAL_VJP_VJP ? out_grad_grad_hidden : nullptr, wgrad ? workspace : nullptr,
               edges, tiles, num_basis, scale};
  if (edges > 0) {
    const dim3 grid(static_cast<unsigned>(wgrad ? blocks : (tiles + kRWaves - 1) / kRWaves)), block(kRThreads);
    if (mode == ICTC_RADIAL_VALUE)
      hipLaunchKernelGGL((radial_mlp_kernel<ICTC_RADIAL_VALUE, false>), grid, block, 0, stream, a);
    else if (mode == ICTC_RADIAL_VJP && wgrad)
      hipLaunchKernelGGL((radial_mlp_kernel<ICTC_RADIAL_VJP, true>), grid, block, 0, stream, a);
    else if (mode == ICTC_RADIAL_VJP)
      hipLaunchKernelGGL((radial_mlp_kernel<ICTC_RADIAL_VJP, false>), grid, block, 0, stream, a);
    else if (wgrad)
      hipLaunchKernelGGL((radial_mlp_kernel<ICTC_RADIAL_VJP_VJP, true>), grid, block, 0, stream, a);
    else
      hipLaunchKernelGGL((radial_mlp_kernel<ICTC_RADIAL_VJP_VJP, false>), grid, block, 0, stream, a);
    if (hipGetLastError() != hipSuccess) return ICTC_ERR_LAUNCH;
  }
  if (wgrad) {
    hipLaunchKernelGGL(radial_wsum_kernel, dim3(kPart / kSumRows), dim3(256), 0, stream, workspace, blocks, num_basis,
                       scale, grad_w1, grad_w2, grad_w3);
    if (hipGetLastError() != hipSuccess) return ICTC_ERR_LAUNCH;
  }
  return ICTC_OK;
}
