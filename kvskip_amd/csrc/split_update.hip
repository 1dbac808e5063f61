// The split pass carrying another layer's update over a contiguous cache; the kernels are in
// split_update.hpp, the paged-cache ones in split_update_paged.hip.
#include "split_update.hpp"

namespace kvs {

hipError_t launch_split_update(const AttnP& a, const kvskip_update_args& u, int D, hipStream_t s) {
  const int G = a.Hq / a.Hkv;
  const int nb = (u.T + BLK - 1) / BLK;
  if (!qk_use_mfma() || nb > CARRY_MAX_R * WAVE || G != u.Hq / u.Hkv) {  // two launches, same results
    const hipError_t e = launch_update(u, s);
    if (e != hipSuccess) return e;
    return launch_decode(a, D, G, true, true, true, 1, s);
  }
  if (a.block_table != nullptr) return launch_split_update_paged(a, u, D, s);
#define KVS_CASE(DD, GG) \
  if (D == DD && G == GG) return launch_split_update_g<DD, GG, false>(a, u, s);
  KVS_FOR_G(KVS_CASE, 64)
  KVS_FOR_G(KVS_CASE, 128)
#undef KVS_CASE
  return hipErrorInvalidValue;
}

}  // namespace kvs
