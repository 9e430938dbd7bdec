// lanes.h -- sums over aligned groups of L lanes of a wave (internal).
#pragma once

#include <hip/hip_runtime.h>

namespace ien {

// v from lane (lane's row of 16, pattern CTRL): a DPP move, no LDS trip.
template <int CTRL>
__device__ __forceinline__ float dpp_from(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// The sum of v over each aligned group of L lanes (L a power of two up to
// 64), in every lane of the group: lanes xor 1 and xor 2 by quad
// permutations, then the other quad of 8 by the half-row mirror and the
// other half of 16 by the row mirror (each pairs every lane with a lane of
// the other part, whose value by then is that part's sum); across rows of
// 16 and halves of 32 by lane shuffles.  Lanes outside the group's range
// are never read, so groups may be active or not independently.
template <int L>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (L >= 2) v += dpp_from<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  if constexpr (L >= 4) v += dpp_from<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  if constexpr (L >= 8) v += dpp_from<0x141>(v);  // row_half_mirror
  if constexpr (L >= 16) v += dpp_from<0x140>(v); // row_mirror
  if constexpr (L >= 32) v += __shfl_xor(v, 16);
  if constexpr (L >= 64) v += __shfl_xor(v, 32);
  return v;
}

}  // namespace ien
