// The planner's split pass carrying the update of another (finished) attention layer: one launch
// whose first B' Hkv' workgroups run that update and the rest the masked + statistics split pass
// (MFMA engine) of this layer. The update only needs its own layer's statistics, which the
// earlier pass wrote, and its result is only read by that layer's next plan, so it can ride on
// any later pass; with the update workgroups dispatched first its latency chain runs under the
// pass's streaming instead of in a launch of its own. A group of G > 4 query heads runs two heads
// per wavefront (the pass's workgroups have 4).
#pragma once
#include "attn_decode.hpp"

namespace kvs {
namespace {

template <int D, int G, bool RAG, int R, bool PAGED>
__global__ void __launch_bounds__(NT, 2) split_update_kernel(const AttnP a, const kvskip_update_args u) {
  const int n_update = u.B * u.Hkv;
  const int i = blockIdx.x;
  if (i < n_update)
    update_body<G, R, carry_waves(G)>(u, i % u.Hkv, i / u.Hkv);
  else
    decode_body<D, G, true, true, true, true, RAG, false, PAGED>(a, i - n_update);
}

template <int D, int G, bool RAG, bool PAGED>
hipError_t launch_split_update_t(const AttnP& a, const kvskip_update_args& u, hipStream_t s) {
  const int nb = (u.T + BLK - 1) / BLK;
  const dim3 grid(attn_grid(a).x + u.B * u.Hkv), blk(NT);
  if (nb <= 2 * WAVE) hipLaunchKernelGGL((split_update_kernel<D, G, RAG, 2, PAGED>), grid, blk, 0, s, a, u);
  else if (nb <= 4 * WAVE) hipLaunchKernelGGL((split_update_kernel<D, G, RAG, 4, PAGED>), grid, blk, 0, s, a, u);
  else if (nb <= 8 * WAVE) hipLaunchKernelGGL((split_update_kernel<D, G, RAG, 8, PAGED>), grid, blk, 0, s, a, u);
  else if (nb <= 16 * WAVE) hipLaunchKernelGGL((split_update_kernel<D, G, RAG, 16, PAGED>), grid, blk, 0, s, a, u);
  else hipLaunchKernelGGL((split_update_kernel<D, G, RAG, CARRY_MAX_R, PAGED>), grid, blk, 0, s, a, u);
  return hipGetLastError();
}

template <int D, int G, bool PAGED>
hipError_t launch_split_update_g(const AttnP& a, const kvskip_update_args& u, hipStream_t s) {
  return a.seq_lens != nullptr ? launch_split_update_t<D, G, true, PAGED>(a, u, s)
                               : launch_split_update_t<D, G, false, PAGED>(a, u, s);
}

}  // namespace
}  // namespace kvs
