// Edge embedding of the MACE interaction in one pass per derivative order (gfx950).
//
// From the edge vector v (r = |v|) the model forms
//   n      = v / max(r, 1e-8)                                   (the direction fed to the harmonics)
//   emb_b  = sqrt(2 / r_max) sin(b pi r / r_max) / max(r, 1e-12) * u(r / r_max),   b = 1..B
//   u(x)   = 1 - (p+1)(p+2)/2 x^p + p(p+2) x^(p+1) - p(p+1)/2 x^(p+2)   for r < r_max, 0 beyond
// (reference mace_ictc/models/pure_cartesian_ictd_fix.py:2930-2950 for n and r,
// mace_ictc/models/radial_basis.py:11-92 for the Bessel basis and the polynomial cutoff), where a
// composition of library ops takes some twenty passes over [E, 3] and [E, B] tensors per order.
// Modes (f = (n, emb), one thread per edge, every derivative analytic):
//   VALUE: (n [E,3], emb [E,B])
//   VJP  : d<(gn, ge), f>/dv                           [E,3]   (gn or ge may be null: zero)
//   JVP  : (df_n[t], df_emb[t])                        [E,3], [E,B]   (either output may be null)
//   HVP  : d/dv <(gn, ge), df[t]> = d/dv of the VJP along t   [E,3]
// With rhat = v / r and the tangent's projection t_perp = (t - (rhat.t) rhat) / r:
//   VJP  = (gn - (gn.n) n) / r + S1 rhat,                S1 = sum_b ge_b emb_b'(r)
//   JVP  = (t_perp, emb_b'(r) (rhat.t))
//   HVP  = -gn (n.t) / r^2 - (gn.t_perp) n / r - (gn.n) t_perp / r + (gn.n)(n.t) n / r^2
//          + S2 (rhat.t) rhat + S1 t_perp,               S2 = sum_b ge_b emb_b''(r)
// For r < 1e-8 the direction is v / 1e-8 (the clamp's constant branch: derivative I / 1e-8, no
// curvature); for r = 0 the radial terms' derivatives are taken as zero.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "ictc_hip.h"

namespace ictc {
namespace {

constexpr int kGeoBlock = 256;
constexpr float kDirFloor = 1e-8f;
constexpr float kRadFloor = 1e-12f;

struct EmbeddingArgs {
  int basis;       // B
  int p;           // cutoff power
  float r_max;
};

// emb_b(r) and its first two derivatives in r (d1, d2 only when requested).
struct RadialValue {
  float f, d1, d2;
};

// u(r / r_max) and its first two derivatives in r; zero from r_max on.
__device__ __forceinline__ void envelope(float r, const EmbeddingArgs& a, float& u, float& u1, float& u2) {
  if (!(r < a.r_max)) {
    u = u1 = u2 = 0.f;
    return;
  }
  const float x = r / a.r_max;
  const float p = static_cast<float>(a.p);
  const float c1 = (p + 1.f) * (p + 2.f) * 0.5f, c2 = p * (p + 2.f), c3 = p * (p + 1.f) * 0.5f;
  float xp2 = 1.f;                                   // x^(p-2), built by repeated products
  for (int i = 2; i < a.p; ++i) xp2 *= x;
  const float xp1 = a.p >= 2 ? xp2 * x : 1.f;        // x^(p-1)
  const float xp = a.p >= 1 ? (a.p >= 2 ? xp1 * x : x) : 1.f;   // x^p
  u = 1.f - c1 * xp + c2 * xp * x - c3 * xp * x * x;
  const float inv = 1.f / a.r_max;
  u1 = inv * (-c1 * p * (a.p >= 1 ? xp1 : 0.f) + c2 * (p + 1.f) * xp - c3 * (p + 2.f) * xp * x);
  u2 = inv * inv *
       (-c1 * p * (p - 1.f) * (a.p >= 2 ? xp2 : 0.f) + c2 * (p + 1.f) * p * (a.p >= 1 ? xp1 : 0.f) -
        c3 * (p + 2.f) * (p + 1.f) * xp);
}

// Bessel term b (1-based) times the envelope, with derivatives.
__device__ __forceinline__ RadialValue radial(int b, float r, float u, float u1, float u2, const EmbeddingArgs& a) {
  const float A = sqrtf(2.f / a.r_max);
  const float w = static_cast<float>(b) * (3.14159265358979323846f / a.r_max);
  float s, c;
  sincosf(w * r, &s, &c);
  const float rd = fmaxf(r, kRadFloor);
  const float inv = 1.f / rd;
  const float e = A * s * inv;                                   // sin(w r) / r
  const float e1 = A * (w * c - s * inv) * inv;                  // its derivative
  const float e2 = A * (-w * w * s - 2.f * w * c * inv + 2.f * s * inv * inv) * inv;
  RadialValue v;
  v.f = e * u;
  v.d1 = e1 * u + e * u1;
  v.d2 = e2 * u + 2.f * e1 * u1 + e * u2;
  return v;
}

template <int MODE>
__global__ void __launch_bounds__(kGeoBlock)
edge_embedding_kernel(const float* __restrict__ vec, const float* __restrict__ gn, const float* __restrict__ ge,
                      const float* __restrict__ t, float* __restrict__ out_a, float* __restrict__ out_b,
                      const EmbeddingArgs a, int64_t edges) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kGeoBlock;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * kGeoBlock + threadIdx.x; e < edges; e += stride) {
    const float vx = vec[3 * e], vy = vec[3 * e + 1], vz = vec[3 * e + 2];
    const float r = sqrtf(vx * vx + vy * vy + vz * vz);
    const bool dir_live = r >= kDirFloor;                 // the direction's clamp is inactive
    const float c = dir_live ? r : kDirFloor;
    const float nx = vx / c, ny = vy / c, nz = vz / c;
    const float ir = r > 0.f ? 1.f / r : 0.f;
    const float hx = vx * ir, hy = vy * ir, hz = vz * ir;   // rhat (0 for r = 0)
    float u, u1, u2;
    envelope(r, a, u, u1, u2);
    if constexpr (MODE == ICTC_EMBED_VALUE) {
      out_a[3 * e] = nx;
      out_a[3 * e + 1] = ny;
      out_a[3 * e + 2] = nz;
      for (int b = 0; b < a.basis; ++b) out_b[e * a.basis + b] = radial(b + 1, r, u, u1, u2, a).f;
    } else if constexpr (MODE == ICTC_EMBED_VJP) {
      float ox = 0.f, oy = 0.f, oz = 0.f;
      if (gn != nullptr) {
        const float gx = gn[3 * e], gy = gn[3 * e + 1], gz = gn[3 * e + 2];
        if (dir_live) {
          const float dot = gx * nx + gy * ny + gz * nz;
          ox = (gx - dot * nx) * ir;
          oy = (gy - dot * ny) * ir;
          oz = (gz - dot * nz) * ir;
        } else {
          ox = gx / kDirFloor;
          oy = gy / kDirFloor;
          oz = gz / kDirFloor;
        }
      }
      if (ge != nullptr) {
        float s1 = 0.f;
        for (int b = 0; b < a.basis; ++b) s1 = fmaf(ge[e * a.basis + b], radial(b + 1, r, u, u1, u2, a).d1, s1);
        ox = fmaf(s1, hx, ox);
        oy = fmaf(s1, hy, oy);
        oz = fmaf(s1, hz, oz);
      }
      out_a[3 * e] = ox;
      out_a[3 * e + 1] = oy;
      out_a[3 * e + 2] = oz;
    } else if constexpr (MODE == ICTC_EMBED_JVP) {
      const float tx = t[3 * e], ty = t[3 * e + 1], tz = t[3 * e + 2];
      if (out_a != nullptr) {
        if (dir_live) {
          const float dot = nx * tx + ny * ty + nz * tz;
          out_a[3 * e] = (tx - dot * nx) * ir;
          out_a[3 * e + 1] = (ty - dot * ny) * ir;
          out_a[3 * e + 2] = (tz - dot * nz) * ir;
        } else {
          out_a[3 * e] = tx / kDirFloor;
          out_a[3 * e + 1] = ty / kDirFloor;
          out_a[3 * e + 2] = tz / kDirFloor;
        }
      }
      if (out_b != nullptr) {
        const float ht = hx * tx + hy * ty + hz * tz;
        for (int b = 0; b < a.basis; ++b) out_b[e * a.basis + b] = radial(b + 1, r, u, u1, u2, a).d1 * ht;
      }
    } else {   // HVP
      const float tx = t[3 * e], ty = t[3 * e + 1], tz = t[3 * e + 2];
      const float ht = hx * tx + hy * ty + hz * tz;
      // t_perp = (t - (rhat.t) rhat) / r  (equal to the direction's JVP when the clamp is inactive)
      const float px = (tx - ht * hx) * ir, py = (ty - ht * hy) * ir, pz = (tz - ht * hz) * ir;
      float ox = 0.f, oy = 0.f, oz = 0.f;
      if (gn != nullptr && dir_live) {
        const float gx = gn[3 * e], gy = gn[3 * e + 1], gz = gn[3 * e + 2];
        const float gnn = gx * nx + gy * ny + gz * nz;
        const float gp = gx * px + gy * py + gz * pz;
        const float nt = ht;                     // n = rhat when the clamp is inactive
        const float ir2 = ir * ir;
        ox = -gx * nt * ir2 - gp * nx * ir - gnn * px * ir + gnn * nt * nx * ir2;
        oy = -gy * nt * ir2 - gp * ny * ir - gnn * py * ir + gnn * nt * ny * ir2;
        oz = -gz * nt * ir2 - gp * nz * ir - gnn * pz * ir + gnn * nt * nz * ir2;
      }
      if (ge != nullptr) {
        float s1 = 0.f, s2 = 0.f;
        for (int b = 0; b < a.basis; ++b) {
          const RadialValue v = radial(b + 1, r, u, u1, u2, a);
          const float g = ge[e * a.basis + b];
          s1 = fmaf(g, v.d1, s1);
          s2 = fmaf(g, v.d2, s2);
        }
        ox += s2 * ht * hx + s1 * px;
        oy += s2 * ht * hy + s1 * py;
        oz += s2 * ht * hz + s1 * pz;
      }
      out_a[3 * e] = ox;
      out_a[3 * e + 1] = oy;
      out_a[3 * e + 2] = oz;
    }
  }
}

}  // namespace
}  // namespace ictc

extern "C" int ictc_hip_edge_embedding(int mode, const float* vectors, const float* grad_directions,
                                       const float* grad_embedding, const float* tangent, float* out_directions,
                                       float* out_embedding, int num_basis, int cutoff_p, float r_max,
                                       int64_t edges, hipStream_t stream) {
  using namespace ictc;
  if (edges < 0 || num_basis < 1 || num_basis > ICTC_EMBED_MAX_BASIS || cutoff_p < 1 ||
      cutoff_p > ICTC_EMBED_MAX_POWER || !(r_max > 0.f))
    return ICTC_ERR_INVALID_ARGUMENT;
  if (edges == 0) return ICTC_OK;
  if (vectors == nullptr) return ICTC_ERR_INVALID_ARGUMENT;
  switch (mode) {
    case ICTC_EMBED_VALUE:
      if (!out_directions || !out_embedding) return ICTC_ERR_INVALID_ARGUMENT;
      break;
    case ICTC_EMBED_VJP:
      if (!out_directions) return ICTC_ERR_INVALID_ARGUMENT;
      break;
    case ICTC_EMBED_JVP:
      if (!tangent) return ICTC_ERR_INVALID_ARGUMENT;
      if (!out_directions && !out_embedding) return ICTC_OK;
      break;
    case ICTC_EMBED_HVP:
      if (!tangent || !out_directions) return ICTC_ERR_INVALID_ARGUMENT;
      break;
    default:
      return ICTC_ERR_INVALID_ARGUMENT;
  }
  const EmbeddingArgs a{num_basis, cutoff_p, r_max};
  const int64_t blocks = (edges + kGeoBlock - 1) / kGeoBlock;
  const dim3 grid(static_cast<unsigned>(blocks < 16384 ? blocks : 16384));
  switch (mode) {
    case ICTC_EMBED_VALUE:
      hipLaunchKernelGGL(edge_embedding_kernel<ICTC_EMBED_VALUE>, grid, dim3(kGeoBlock), 0, stream, vectors,
                         grad_directions, grad_embedding, tangent, out_directions, out_embedding, a, edges);
      break;
    case ICTC_EMBED_VJP:
      hipLaunchKernelGGL(edge_embedding_kernel<ICTC_EMBED_VJP>, grid, dim3(kGeoBlock), 0, stream, vectors,
                         grad_directions, grad_embedding, tangent, out_directions, out_embedding, a, edges);
      break;
    case ICTC_EMBED_JVP:
      hipLaunchKernelGGL(edge_embedding_kernel<ICTC_EMBED_JVP>, grid, dim3(kGeoBlock), 0, stream, vectors,
                         grad_directions, grad_embedding, tangent, out_directions, out_embedding, a, edges);
      break;
    default:
      hipLaunchKernelGGL(edge_embedding_kernel<ICTC_EMBED_HVP>, grid, dim3(kGeoBlock), 0, stream, vectors,
                         grad_directions, grad_embedding, tangent, out_directions, out_embedding, a, edges);
      break;
  }
  return hipGetLastError() == hipSuccess ? ICTC_OK : ICTC_ERR_LAUNCH;
}
