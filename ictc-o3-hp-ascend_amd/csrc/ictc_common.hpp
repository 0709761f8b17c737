// Shared device helpers for the ictc_o3 HIP kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ictc_hip.h"

namespace ictc {

constexpr int kWave = 64;

template <int N>
struct Int {
  static constexpr int value = N;
  constexpr operator int() const { return N; }
};

// Compile-time loop: f(Int<B>{}), f(Int<B+1>{}), ..., f(Int<E-1>{}).
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(Int<B>{});
    static_for<B + 1, E>(f);
  }
}

// Full triangle/parity path set of (LIN, LE, LOUT) in ascending (l1,l2,l3) order,
// the enumeration order of the reference owner (ictd_irreps.py:2161-2175).
struct PathTable {
  int n = 0;
  int l1[ICTC_MAX_PATHS] = {};
  int l2[ICTC_MAX_PATHS] = {};
  int l3[ICTC_MAX_PATHS] = {};
  int bond[ICTC_MAX_PATHS] = {};  // first bond entry of the path, M_p stored [k][i]
  int out[ICTC_MAX_PATHS] = {};   // first output component of the path
  int nbond = 0;
  int noc = 0;                    // output components
};

// Output layout: ascending l3, and within one l3 the paths in enumeration order
// (the owner's path_offset: groups sorted by (l1,l2), reference ictd_irreps.py:2514-2526).
constexpr PathTable make_paths(int lin, int le, int lout) {
  PathTable t{};
  for (int a = 0; a <= lin; ++a)
    for (int b = 0; b <= le; ++b)
      for (int c = 0; c <= lout; ++c) {
        const int lo = a > b ? a - b : b - a;
        if (c < lo || c > a + b || ((a + b + c) & 1)) continue;
        t.l1[t.n] = a;
        t.l2[t.n] = b;
        t.l3[t.n] = c;
        t.bond[t.n] = t.nbond;
        t.nbond += (2 * a + 1) * (2 * c + 1);
        ++t.n;
      }
  for (int l = 0; l <= lout; ++l)
    for (int p = 0; p < t.n; ++p)
      if (t.l3[p] == l) {
        t.out[p] = t.noc;
        t.noc += 2 * l + 1;
      }
  return t;
}

template <int LIN, int LE, int LOUT>
struct Paths {
  static constexpr PathTable tab = make_paths(LIN, LE, LOUT);
  static constexpr int N = tab.n;
  static constexpr int NB = tab.nbond;
  static constexpr int NOC = tab.noc;
  static constexpr int NX = (LIN + 1) * (LIN + 1);
  static constexpr int NY = (LE + 1) * (LE + 1);
};

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Vector of NV consecutive floats: one global load/store instruction per lane.
template <int NV>
struct Vec {
  float v[NV];
};

template <int NV>
__device__ __forceinline__ Vec<NV> load_vec(const float* __restrict__ p) {
  Vec<NV> r;
  if constexpr (NV == 1) {
    r.v[0] = p[0];
  } else if constexpr (NV == 2) {
    const f32x2 t = *reinterpret_cast<const f32x2*>(p);
    r.v[0] = t.x;
    r.v[1] = t.y;
  } else {
    static_assert(NV == 4, "NV must be 1, 2 or 4");
    const f32x4 t = *reinterpret_cast<const f32x4*>(p);
    r.v[0] = t.x;
    r.v[1] = t.y;
    r.v[2] = t.z;
    r.v[3] = t.w;
  }
  return r;
}

// Streaming store: the outputs are written once and not re-read by this kernel.
template <int NV>
__device__ __forceinline__ void store_vec_nt(float* __restrict__ p, const Vec<NV>& r) {
  if constexpr (NV == 1) {
    __builtin_nontemporal_store(r.v[0], p);
  } else if constexpr (NV == 2) {
    f32x2 t = {r.v[0], r.v[1]};
    __builtin_nontemporal_store(t, reinterpret_cast<f32x2*>(p));
  } else {
    f32x4 t = {r.v[0], r.v[1], r.v[2], r.v[3]};
    __builtin_nontemporal_store(t, reinterpret_cast<f32x4*>(p));
  }
}

template <int NV>
__device__ __forceinline__ void store_vec(float* __restrict__ p, const Vec<NV>& r) {
  if constexpr (NV == 1) {
    p[0] = r.v[0];
  } else if constexpr (NV == 2) {
    *reinterpret_cast<f32x2*>(p) = f32x2{r.v[0], r.v[1]};
  } else {
    *reinterpret_cast<f32x4*>(p) = f32x4{r.v[0], r.v[1], r.v[2], r.v[3]};
  }
}

// Returns p unchanged, but opaque to the optimiser: reads through the result cannot
// be hoisted out of the enclosing loop iteration (keeps per-instance LDS tables from
// being promoted wholesale into registers).
__device__ __forceinline__ const float* opaque_lds_row(const float* p) {
  uint32_t off = 0;
  asm volatile("" : "+s"(off));
  return p + off;
}

// ---------------------------------------------------------------- buffer resources
// Raw buffer descriptors (base in SGPRs, 32-bit offsets, hardware range check on
// num_records).  A descriptor over a null pointer gets num_records = 0: its loads
// return 0 and its stores are discarded, which is how optional outputs are skipped
// without branches.
using rsrc_t = __amdgpu_buffer_rsrc_t;
constexpr int kRsrcWord3 = 0x00020000;  // gfx9-family raw buffer, 32-bit dwords
constexpr int kNonTemporal = 2;         // nt cache-policy bit

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, base ? bytes : 0u, kRsrcWord3);
}

// The whole byte offset goes into the per-lane voffset (soffset = 0): the range check
// then compares exactly that offset with num_records.  `policy` is the cache-policy
// operand (0 = default; kNonTemporal for rows read exactly once).
template <int NV, int policy = 0>
__device__ __forceinline__ Vec<NV> buf_load(rsrc_t r, uint32_t off) {
  const uint32_t voff = off, soff = 0;
  Vec<NV> out;
  if constexpr (NV == 1) {
    out.v[0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, policy));
  } else if constexpr (NV == 2) {
    const f32x2 t = __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, policy));
    out.v[0] = t.x;
    out.v[1] = t.y;
  } else {
    const f32x4 t = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, policy));
    out.v[0] = t.x;
    out.v[1] = t.y;
    out.v[2] = t.z;
    out.v[3] = t.w;
  }
  return out;
}

// One float at voffset + soffset, with a wave-uniform soffset (an SGPR, so no per-load
// VGPR).  The range check covers voffset only: callers keep voffset + soffset inside
// the descriptor's range themselves (soffset below a row, lanes clamped to a real
// channel) and put anything data-dependent in voffset.
template <int policy = 0>
__device__ __forceinline__ float buf_load_vs(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, policy));
}

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int NV, int policy = kNonTemporal>
__device__ __forceinline__ void buf_store(rsrc_t r, uint32_t off, const Vec<NV>& v) {
  const uint32_t voff = off, soff = 0;
  if constexpr (NV == 1) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned int, v.v[0]), r, voff, soff, policy);
  } else if constexpr (NV == 2) {
    const f32x2 t = {v.v[0], v.v[1]};
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, t), r, voff, soff, policy);
  } else {
    const f32x4 t = {v.v[0], v.v[1], v.v[2], v.v[3]};
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, t), r, voff, soff, policy);
  }
}

// Branch-free per-lane row store: value v of channel c in row r of a [rows][C] block at
// rsrc r (num_records = rows * C * 4).  Lanes past C get an offset beyond num_records, so
// the hardware drops their store; no divergent branch (into which the compiler would sink
// the arithmetic feeding the store) is needed.
__device__ __forceinline__ void buf_store_lane(rsrc_t r, bool live, uint32_t off, float v) {
  buf_store<1>(r, live ? off : 0xFFFFFFF0u, Vec<1>{{v}});
}

// Compute units of the current device (256 on MI355X), read once per device.
inline int compute_units() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    cached[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
  }
  return cached[dev];
}

// Workgroups are dispatched to the GPU's XCDs (each with its own L2) round-robin by block
// index.  xcd_block(b, n) renumbers the n blocks of a launch so that each XCD receives one
// contiguous range of work items (XCD x gets items [start(x), start(x) + count(x))), which
// keeps neighbouring items -- e.g. receivers of a spatially ordered graph, whose source rows
// overlap -- in the same L2.  A bijection on [0, n).
constexpr int kXcds = 8;

__device__ __forceinline__ uint32_t xcd_block(uint32_t b, uint32_t n) {
  const uint32_t q = n / kXcds, r = n % kXcds;
  const uint32_t x = b % kXcds, i = b / kXcds;
  return x * q + (x < r ? x : r) + i;
}

// Sum over the 64 lanes of a wave; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// Sums over the 64 lanes of N values per lane at once (N <= 16), by a transposing butterfly:
// at each of the first log2(P) exchange distances (32, 16, ...) a lane keeps one half of its
// values and receives its partner's sums of that half, then plain butterflies finish; P - 1 +
// 6 - log2(P) exchanges instead of 6 N (P = N rounded up to a power of two).  Returns the total
// of value index j = (lane >> (6 - log2 P)) & (P - 1) (0 for j >= N); the lanes with
// lane & ((64 >> log2 P) - 1) == 0 hold each index exactly once.
template <int N>
struct WaveSums {
  static constexpr int P = N <= 1 ? 1 : N <= 2 ? 2 : N <= 4 ? 4 : N <= 8 ? 8 : 16;
  static constexpr int LOGP = P == 1 ? 0 : P == 2 ? 1 : P == 4 ? 2 : P == 8 ? 3 : 4;
  static constexpr int SHIFT = 6 - LOGP;
  static_assert(N >= 1 && N <= 16, "WaveSums: 1 <= N <= 16");
  __device__ static __forceinline__ int index(int lane) { return (lane >> SHIFT) & (P - 1); }
  __device__ static __forceinline__ bool owner(int lane) { return (lane & ((1 << SHIFT) - 1)) == 0; }
  __device__ static __forceinline__ float reduce(const float (&v)[N], int lane) {
    float t[P];
#pragma unroll
    for (int i = 0; i < P; ++i) t[i] = i < N ? v[i] : 0.f;
    static_for<0, LOGP>([&](auto S) {
      constexpr int half = P >> (S + 1);
      constexpr int dist = 32 >> S;
      const bool upper = (lane & dist) != 0;
#pragma unroll
      for (int i = 0; i < half; ++i) {
        const float send = upper ? t[i] : t[i + half];
        const float keep = upper ? t[i + half] : t[i];
        t[i] = keep + __shfl_xor(send, dist, kWave);
      }
    });
    float r = t[0];
#pragma unroll
    for (int off = 32 >> LOGP; off > 0; off >>= 1) r += __shfl_xor(r, off, kWave);
    return r;
  }
};

// Channel sums of N per-lane partials (one per harmonic component) stored to N floats at rsrc
// r: one transposing butterfly per group of 16 components.
template <int N>
__device__ __forceinline__ void store_channel_sums(const float (&v)[N], int lane, rsrc_t r) {
  static_for<0, (N + 15) / 16>([&](auto H) {
    constexpr int h0 = 16 * H, nh = N - h0 < 16 ? N - h0 : 16;
    using WS = WaveSums<nh>;
    float part[nh];
#pragma unroll
    for (int j = 0; j < nh; ++j) part[j] = v[h0 + j];
    const float tot = WS::reduce(part, lane);
    const int j = WS::index(lane);
    if (WS::owner(lane) && j < nh) buf_store<1, 0>(r, static_cast<uint32_t>(h0 + j) * 4u, Vec<1>{{tot}});
  });
}

}  // namespace ictc
