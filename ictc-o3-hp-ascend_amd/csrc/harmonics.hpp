// Direction harmonics Y_l(n), l = 0..LMAX, in the ICTC basis, and their analytic
// derivative contractions (gfx950).
//
// Y_l[m](n) = sum_r coef_l[r][m] * x^a_r y^b_r z^c_r over the degree-l monomials r
// (reference ictc_o3/basis/ictd_irreps.py:1113-1168; coef = multinomial * G_l B_l *
// component scale, :891-953).  Every Y_l is a homogeneous polynomial, so for a
// cotangent u the scalar phi_u(n) = sum_lm u_lm Y_lm(n) is the polynomial with
// monomial weights w_r = sum_m u_lm coef_l[r][m], and all derivative contractions
// reduce to derivatives of monomials:
//   VALUE : out[lm] = Y_lm(n)
//   VJP   : out[d]  = d phi_u / d n_d                         (first adjoint)
//   JVP   : out[lm] = sum_d t_d dY_lm/dn_d
//   HVP   : out[d]  = sum_e t_e d2 phi_u / dn_d dn_e           (second adjoint wrt n)
//   JVP2  : out[lm] = sum_de t_d s_e d2 Y_lm / dn_d dn_e
//   T3    : out[d]  = sum_ef t_e s_f d3 phi_u / dn_d dn_e dn_f
// which replaces the generated kernel with analytic first/second adjoints of
// reference ictc_o3/ops/generated_direction_harmonics.py:43-194 and extends it to
// third order.  One thread per direction; rows are independent.
#pragma once
#include "ictc_common.hpp"
#include "generated/ictc_cg_table.hpp"

namespace ictc {

// Exponents of monomial r of degree L in basis row order (a-major, then b).
constexpr int mono_a(int L, int r) {
  int a = 0;
  while (r >= L - a + 1) {
    r -= L - a + 1;
    ++a;
  }
  return a;
}
constexpr int mono_b(int L, int r) {
  int a = 0;
  while (r >= L - a + 1) {
    r -= L - a + 1;
    ++a;
  }
  return r;
}

constexpr float falling(int n, int k) {
  float f = 1.f;
  for (int i = 0; i < k; ++i) f *= static_cast<float>(n - i);
  return f;
}

// d^(i+j+k)/dx^i dy^j dz^k of x^a y^b z^c.
template <int A, int B, int Cc, int I, int J, int K>
__device__ __forceinline__ float dmono(const float* px, const float* py, const float* pz) {
  if constexpr (I > A || J > B || K > Cc) {
    return 0.f;
  } else {
    constexpr float f = falling(A, I) * falling(B, J) * falling(Cc, K);
    return f * px[A - I] * py[B - J] * pz[Cc - K];
  }
}

template <int A, int B, int Cc, int D>
__device__ __forceinline__ float d1(const float* px, const float* py, const float* pz) {
  return dmono<A, B, Cc, D == 0, D == 1, D == 2>(px, py, pz);
}
template <int A, int B, int Cc, int D, int E>
__device__ __forceinline__ float d2(const float* px, const float* py, const float* pz) {
  return dmono<A, B, Cc, (D == 0) + (E == 0), (D == 1) + (E == 1), (D == 2) + (E == 2)>(px, py, pz);
}
template <int A, int B, int Cc, int D, int E, int F>
__device__ __forceinline__ float d3(const float* px, const float* py, const float* pz) {
  return dmono<A, B, Cc, (D == 0) + (E == 0) + (F == 0), (D == 1) + (E == 1) + (F == 1),
               (D == 2) + (E == 2) + (F == 2)>(px, py, pz);
}

template <int LMAX>
__global__ void __launch_bounds__(256)
harmonics_kernel(int mode, const float* __restrict__ n, const float* __restrict__ u,
                 const float* __restrict__ t, const float* __restrict__ s, float* __restrict__ out,
                 int64_t rows) {
  constexpr int NY = (LMAX + 1) * (LMAX + 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (row >= rows) return;
  float px[LMAX + 1], py[LMAX + 1], pz[LMAX + 1];
  px[0] = py[0] = pz[0] = 1.f;
  const float x = n[row * 3 + 0], y = n[row * 3 + 1], z = n[row * 3 + 2];
#pragma unroll
  for (int k = 1; k <= LMAX; ++k) {
    px[k] = px[k - 1] * x;
    py[k] = py[k - 1] * y;
    pz[k] = pz[k - 1] * z;
  }
  float tv[3] = {0.f, 0.f, 0.f}, sv[3] = {0.f, 0.f, 0.f};
  if (mode >= ICTC_HARM_JVP) {
#pragma unroll
    for (int d = 0; d < 3; ++d) tv[d] = t[row * 3 + d];
  }
  if (mode >= ICTC_HARM_JVP2) {
#pragma unroll
    for (int d = 0; d < 3; ++d) sv[d] = s[row * 3 + d];
  }
  const bool per_component = mode == ICTC_HARM_VALUE || mode == ICTC_HARM_JVP || mode == ICTC_HARM_JVP2;
  float acc3[3] = {0.f, 0.f, 0.f};
  static_for<0, LMAX + 1>([&](auto Lc) {
    constexpr int L = Lc;
    constexpr int NM = 2 * L + 1;
    using H = HarmTab<L>;
    float ul[NM];
    float yl[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      ul[m] = per_component ? 0.f : u[row * NY + L * L + m];
      yl[m] = 0.f;
    }
    static_for<0, H::nmono>([&](auto R) {
      constexpr int a = mono_a(L, R), b = mono_b(L, R), c = L - a - b;
      if (per_component) {
        float mv;
        if (mode == ICTC_HARM_VALUE) {
          mv = px[a] * py[b] * pz[c];
        } else if (mode == ICTC_HARM_JVP) {
          mv = d1<a, b, c, 0>(px, py, pz) * tv[0] + d1<a, b, c, 1>(px, py, pz) * tv[1] +
               d1<a, b, c, 2>(px, py, pz) * tv[2];
        } else {
          mv = 0.f;
          static_for<0, 3>([&](auto D) {
            static_for<0, 3>([&](auto E) { mv += d2<a, b, c, D, E>(px, py, pz) * tv[D] * sv[E]; });
          });
        }
        static_for<0, NM>([&](auto M) {
          constexpr float cf = H::coef[R * NM + M];
          if constexpr (cf != 0.0f) yl[M] = fmaf(cf, mv, yl[M]);
        });
      } else {
        float w = 0.f;
        static_for<0, NM>([&](auto M) {
          constexpr float cf = H::coef[R * NM + M];
          if constexpr (cf != 0.0f) w = fmaf(cf, ul[M], w);
        });
        static_for<0, 3>([&](auto D) {
          float g;
          if (mode == ICTC_HARM_VJP) {
            g = d1<a, b, c, D>(px, py, pz);
          } else if (mode == ICTC_HARM_HVP) {
            g = 0.f;
            static_for<0, 3>([&](auto E) { g += d2<a, b, c, D, E>(px, py, pz) * tv[E]; });
          } else {
            g = 0.f;
            static_for<0, 3>([&](auto E) {
              static_for<0, 3>([&](auto F) { g += d3<a, b, c, D, E, F>(px, py, pz) * tv[E] * sv[F]; });
            });
          }
          acc3[D] = fmaf(w, g, acc3[D]);
        });
      }
    });
    if (per_component) {
#pragma unroll
      for (int m = 0; m < NM; ++m) out[row * NY + L * L + m] = yl[m];
    }
  });
  if (!per_component) {
#pragma unroll
    for (int d = 0; d < 3; ++d) out[row * 3 + d] = acc3[d];
  }
}

template <int LMAX>
int launch_harmonics(int mode, const float* n, const float* u, const float* t, const float* s,
                     float* out, int64_t rows, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>((rows + 255) / 256));
  hipLaunchKernelGGL(harmonics_kernel<LMAX>, grid, dim3(256), 0, stream, mode, n, u, t, s, out, rows);
  return hipGetLastError() == hipSuccess ? ICTC_OK : ICTC_ERR_LAUNCH;
}

}  // namespace ictc
