// extern "C" entry point of the direction-harmonics family; per-lmax instantiations
// are compiled in generated/harm_inst_*.hip.
#include "harmonics.hpp"

namespace ictc {
#define ICTC_HARM_DECLARE(L)                                                                    \
  extern template int launch_harmonics<L>(int, const float*, const float*, const float*,        \
                                          const float*, float*, int64_t, hipStream_t);
ICTC_HARM_DECLARE(0)
ICTC_HARM_DECLARE(1)
ICTC_HARM_DECLARE(2)
ICTC_HARM_DECLARE(3)
ICTC_HARM_DECLARE(4)
ICTC_HARM_DECLARE(5)
ICTC_HARM_DECLARE(6)
#undef ICTC_HARM_DECLARE
}  // namespace ictc

extern "C" int ictc_hip_direction_harmonics(int lmax, int mode, const float* directions, const float* u,
                                            const float* t, const float* s, float* out, int64_t rows,
                                            hipStream_t stream) {
  if (lmax < 0 || rows < 0 || mode < ICTC_HARM_VALUE || mode > ICTC_HARM_T3) return ICTC_ERR_INVALID_ARGUMENT;
  if (lmax > ICTC_HARM_MAX_LMAX) return ICTC_ERR_UNSUPPORTED;
  if (rows == 0) return ICTC_OK;
  if (!directions || !out) return ICTC_ERR_INVALID_ARGUMENT;
  const bool needs_u = mode == ICTC_HARM_VJP || mode == ICTC_HARM_HVP || mode == ICTC_HARM_T3;
  const bool needs_t = mode >= ICTC_HARM_JVP;
  const bool needs_s = mode >= ICTC_HARM_JVP2;
  if ((needs_u && !u) || (needs_t && !t) || (needs_s && !s)) return ICTC_ERR_INVALID_ARGUMENT;
  using ictc::launch_harmonics;
  switch (lmax) {
    case 0: return launch_harmonics<0>(mode, directions, u, t, s, out, rows, stream);
    case 1: return launch_harmonics<1>(mode, directions, u, t, s, out, rows, stream);
    case 2: return launch_harmonics<2>(mode, directions, u, t, s, out, rows, stream);
    case 3: return launch_harmonics<3>(mode, directions, u, t, s, out, rows, stream);
    case 4: return launch_harmonics<4>(mode, directions, u, t, s, out, rows, stream);
    case 5: return launch_harmonics<5>(mode, directions, u, t, s, out, rows, stream);
    default: return launch_harmonics<6>(mode, directions, u, t, s, out, rows, stream);
  }
}
