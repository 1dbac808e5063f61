// The planned pass over a ragged batch of a contiguous cache (kernels in planned.hpp).
#include "planned.hpp"

namespace kvs {

hipError_t launch_planned_ragged(const AttnP& a, const kvskip_plan_args& pa, const kvskip_update_args* u, int D,
                                 hipStream_t s) {
  const int G = a.Hq / a.Hkv;
#define KVS_CASE(DD, GG) \
  if (D == DD && G == GG) return launch_planned_p<DD, GG, false, true>(a, pa, u, s);
  KVS_FOR_G(KVS_CASE, 64)
  KVS_FOR_G(KVS_CASE, 128)
#undef KVS_CASE
  return hipErrorInvalidValue;
}

}  // namespace kvs
