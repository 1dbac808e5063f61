// The split pass carrying another layer's update over a paged cache (the kernels of
// split_update.hpp with PAGED), compiled apart from the contiguous ones so the two build in parallel.
#include "split_update.hpp"

namespace kvs {

hipError_t launch_split_update_paged(const AttnP& a, const kvskip_update_args& u, int D, hipStream_t s) {
  const int G = a.Hq / a.Hkv;
#define KVS_CASE(DD, GG) \
  if (D == DD && G == GG) return launch_split_update_g<DD, GG, true>(a, u, s);
  KVS_FOR_G(KVS_CASE, 64)
  KVS_FOR_G(KVS_CASE, 128)
#undef KVS_CASE
  return hipErrorInvalidValue;
}

}  // namespace kvs
