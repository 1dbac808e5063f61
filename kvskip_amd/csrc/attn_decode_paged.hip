// The split-K decode pass over a paged KV cache (64-token pages in a pool, a block table per
// sequence): the attention body of attn_decode.hpp with its per-block page resources, for every
// flag combination of the contiguous pass (dense or block lists, statistics, stats-only, fp16 P,
// ragged batches). Kept apart from attn_decode.hip so the two compile in parallel.
#include "attn_decode.hpp"

namespace kvs {
namespace {

template <int D, int G, bool MASKED, bool STATS, bool LOAD_V, bool RAG>
__global__ void __launch_bounds__(NT, 2) decode_paged_kernel(const AttnP p) {
  decode_body<D, G, MASKED, STATS, LOAD_V, true, RAG, false, true>(p, blockIdx.x);
}

template <int D, int G, bool M, bool ST, bool LV>
hipError_t launch_paged_t(const AttnP& p, int phase, hipStream_t s) {
  if (phase & 1) {
    if (p.seq_lens != nullptr)
      hipLaunchKernelGGL((decode_paged_kernel<D, G, M, ST, LV, true>), attn_grid(p), dim3(NT), 0, s, p);
    else
      hipLaunchKernelGGL((decode_paged_kernel<D, G, M, ST, LV, false>), attn_grid(p), dim3(NT), 0, s, p);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if ((phase & 2) && p.num_splits > 1) return launch_combine(p, D, false, s);
  return hipSuccess;
}

template <int D, int G>
hipError_t paged_flags(const AttnP& p, bool masked, bool stats, bool load_v, int phase, hipStream_t s) {
  if (!masked && !stats && load_v) return launch_paged_t<D, G, false, false, true>(p, phase, s);
  if (!masked && stats && load_v) return launch_paged_t<D, G, false, true, true>(p, phase, s);
  if (!masked && stats && !load_v) return launch_paged_t<D, G, false, true, false>(p, phase, s);
  if (masked && !stats && load_v) return launch_paged_t<D, G, true, false, true>(p, phase, s);
  if (masked && stats && load_v) return launch_paged_t<D, G, true, true, true>(p, phase, s);
  if (masked && stats && !load_v) return launch_paged_t<D, G, true, true, false>(p, phase, s);
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_decode_paged(const AttnP& p, int D, int G, bool masked, bool stats, bool load_v, int phase,
                               hipStream_t s) {
#define KVS_CASE(DD, GG) \
  if (D == DD && G == GG) return paged_flags<DD, GG>(p, masked, stats, load_v, phase, s);
  KVS_FOR_G(KVS_CASE, 64)
  KVS_FOR_G(KVS_CASE, 128)
#undef KVS_CASE
  return hipErrorInvalidValue;
}

}  // namespace kvs
