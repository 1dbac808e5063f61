// The planned pass over a paged cache (the kernels of planned.hpp with PAGED), compiled apart from
// the contiguous ones so the two build in parallel. A carried update too long for the fused form has
// already been launched on its own by launch_planned_split (u is then null).
#include "planned.hpp"

namespace kvs {

hipError_t launch_planned_paged(const AttnP& a, const kvskip_plan_args& pa, const kvskip_update_args* u, int D,
                                hipStream_t s) {
  const int G = a.Hq / a.Hkv;
#define KVS_CASE(DD, GG) \
  if (D == DD && G == GG) return launch_planned_p<DD, GG, true>(a, pa, u, s);
  KVS_FOR_G(KVS_CASE, 64)
  KVS_FOR_G(KVS_CASE, 128)
#undef KVS_CASE
  return hipErrorInvalidValue;
}

}  // namespace kvs
