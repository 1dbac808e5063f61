// Split-K decode attention kernels (dense or over block lists, optional per-block statistics,
// stats-only, fp16 P) and their launchers; the workgroup body is in attn_decode.hpp.
#include "attn_decode.hpp"

namespace kvs {
namespace {

template <int D, int G, bool MASKED, bool STATS, bool LOAD_V, bool MF, bool RAG>
__global__ void __launch_bounds__(NT, 2) decode_kernel(const AttnP p) {
  decode_body<D, G, MASKED, STATS, LOAD_V, MF, RAG>(p, blockIdx.x);
}

template <int D, int G, bool M, bool ST, bool LV>
hipError_t launch_decode_t(const AttnP& p, bool mf, int phase, hipStream_t s) {
  if (phase & 1) {
    if (p.block_table != nullptr)  // paged cache: MFMA engine (checked by the caller), own translation unit
      return launch_decode_paged(p, D, G, M, ST, LV, phase, s);
    if (p.seq_lens != nullptr)  // ragged batches: MFMA engine only
      hipLaunchKernelGGL((decode_kernel<D, G, M, ST, LV, true, true>), attn_grid(p), dim3(NT), 0, s, p);
    else if (mf)
      hipLaunchKernelGGL((decode_kernel<D, G, M, ST, LV, true, false>), attn_grid(p), dim3(NT), 0, s, p);
    else
      hipLaunchKernelGGL((decode_kernel<D, G, M, ST, LV, false, false>), attn_grid(p), dim3(NT), 0, s, p);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if ((phase & 2) && p.num_splits > 1) return launch_combine(p, D, false, s);
  return hipSuccess;
}

template <int D, int G>
hipError_t dispatch_flags(const AttnP& p, bool masked, bool stats, bool load_v, bool mf, int phase, hipStream_t s) {
  if (!masked && !stats && load_v) return launch_decode_t<D, G, false, false, true>(p, mf, phase, s);
  if (!masked && stats && load_v) return launch_decode_t<D, G, false, true, true>(p, mf, phase, s);
  if (!masked && stats && !load_v) return launch_decode_t<D, G, false, true, false>(p, mf, phase, s);
  if (masked && !stats && load_v) return launch_decode_t<D, G, true, false, true>(p, mf, phase, s);
  if (masked && stats && load_v) return launch_decode_t<D, G, true, true, true>(p, mf, phase, s);
  if (masked && stats && !load_v) return launch_decode_t<D, G, true, true, false>(p, mf, phase, s);
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_decode(const AttnP& p, int D, int G, bool masked, bool stats, bool load_v, int phase,
                         hipStream_t s) {
  const bool mf = qk_use_mfma();
#define KVS_CASE(DD, GG) \
  if (D == DD && G == GG) return dispatch_flags<DD, GG>(p, masked, stats, load_v, mf, phase, s);
  KVS_FOR_G(KVS_CASE, 64)
  KVS_FOR_G(KVS_CASE, 128)
#undef KVS_CASE
  return hipErrorInvalidValue;
}

}  // namespace kvs
