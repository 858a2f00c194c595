// oxs_stream.hip — launches of the stream kernel (oxs_sampler_dev.h), the
// first of the sampler's two launches.
#include <type_traits>

#include "oxs_sampler_dev.h"

namespace oxs {

template <int DT, int SLOTS, bool VEC, bool MASK>
static hipError_t launch_stream(const Params& p, uint32_t grid, hipStream_t st) {
  const uint32_t* hl = (const uint32_t*)p.history_len;
  const uint32_t* h = (const uint32_t*)p.history;
  const uint32_t hld = (uint32_t)p.history_ld, ld = (uint32_t)p.ld;
  const uint32_t kflags = ((p.flags & OXS_FLAG_SHARED_CONFIG) ? kKShared : 0u) |
                          ((p.flags & kFlagDecode) ? kKDecode : 0u) | ((h && hl) ? kKHistory : 0u) |
                          (p.bias_ids ? kKBias : 0u) | (p.ban_ids ? kKBan : 0u);
  if (p.logits_out)
    hipLaunchKernelGGL((stream_kernel<DT, SLOTS, VEC, MASK, true>), dim3(grid), dim3(kThreads), 0, st, p.logits,
                       p.configs, hl, h, ld, p.S, p.rpx, p.V, kflags, hld, p);
  else
    hipLaunchKernelGGL((stream_kernel<DT, SLOTS, VEC, MASK, false>), dim3(grid), dim3(kThreads), 0, st, p.logits,
                       p.configs, hl, h, ld, p.S, p.rpx, p.V, kflags, hld, p);
  return hipGetLastError();
}

template <int DT, bool VEC, bool MASK>
static hipError_t launch_slots(int slots, const Params& p, uint32_t grid, hipStream_t st) {
  switch (slots) {
    case 8:
      if constexpr (kind_f32(DT)) return launch_stream<DT, 8, VEC, MASK>(p, grid, st);
      return hipErrorInvalidValue;  // bf16 chunks stop at 4 slots (8192 logits)
    case 4: return launch_stream<DT, 4, VEC, MASK>(p, grid, st);
    case 2: return launch_stream<DT, 2, VEC, MASK>(p, grid, st);
    default: return launch_stream<DT, 1, VEC, MASK>(p, grid, st);
  }
}


hipError_t launch_stream_kind(int kind, int slots, bool vec, bool mask, const Params& p, uint32_t grid,
                              hipStream_t st) {
  constexpr int F = OXS_DTYPE_F32, H = OXS_DTYPE_BF16, S = kKindSoftcap;
  auto go = [&](auto kt) -> hipError_t {
    constexpr int SK = decltype(kt)::value;
    if (vec) return mask ? launch_slots<SK, true, true>(slots, p, grid, st) : launch_slots<SK, true, false>(slots, p, grid, st);
    return mask ? launch_slots<SK, false, true>(slots, p, grid, st) : launch_slots<SK, false, false>(slots, p, grid, st);
  };
  switch (kind & ~kKindDecode) {  // the stream kernel has no decode kind
    case F: return go(std::integral_constant<int, F>{});
    case H: return go(std::integral_constant<int, H>{});
    case F | S: return go(std::integral_constant<int, F | S>{});
    case H | S: return go(std::integral_constant<int, H | S>{});
    default: return hipErrorInvalidValue;
  }
}

}  // namespace oxs
