// The planned pass over a contiguous cache; the kernels are in planned.hpp, the paged-cache ones
// in planned_paged.hip.
#include "planned.hpp"

namespace kvs {

hipError_t launch_planned_split(const AttnP& a, const kvskip_plan_args& pa, const kvskip_update_args* u, int D,
                                hipStream_t s) {
  const int G = a.Hq / a.Hkv;
  if (u != nullptr && ((u->T + BLK - 1) / BLK > CARRY_MAX_R * WAVE || G != u->Hq / u->Hkv)) {
    const hipError_t e = launch_update(*u, s);  // the update on its own first, same results
    if (e != hipSuccess) return e;
    u = nullptr;
  }
  if (a.block_table != nullptr) return launch_planned_paged(a, pa, u, D, s);
  if (a.seq_lens != nullptr && a.B > 1) return launch_planned_ragged(a, pa, u, D, s);
#define KVS_CASE(DD, GG) \
  if (D == DD && G == GG) return launch_planned_p<DD, GG, false>(a, pa, u, s);
  KVS_FOR_G(KVS_CASE, 64)
  KVS_FOR_G(KVS_CASE, 128)
#undef KVS_CASE
  return hipErrorInvalidValue;
}

}  // namespace kvs
