// The planner's masked statistics pass with the plan's decision inside: every workgroup's
// prologue merges the scores pass's partials of its (b, KV head), decides as plan_decide does and
// takes its slice of the block list from the chunk masks (decode_body PLANNED), so a layer-step is
// scores -> this pass -> merge, one launch fewer; the first workgroups may carry the update of
// another layer (as kvskip_decode_splits_update).
#pragma once
#include "attn_decode.hpp"

namespace kvs {
namespace {

// The planned pass: the decision of plan_decide made in every workgroup's prologue (decode_body
// PLANNED), optionally with a carried update (R > 0) in the first workgroups.
template <int D, int G, int R, bool PAGED, bool RAG = false>
__global__ void __launch_bounds__(NT, 2) planned_split_kernel(const AttnP a, const kvskip_plan_args pa,
                                                              const kvskip_update_args u) {
  prefetch_planned_args<(R > 0)>();  // the update's arguments only where it is carried
  const int n_update = R > 0 ? u.B * u.Hkv : 0;
  const int i = blockIdx.x;
  if constexpr (R > 0) {
    if (i < n_update) {
      update_body<G, R, carry_waves(G)>(u, i % u.Hkv, i / u.Hkv);
      return;
    }
  }
  decode_body<D, G, true, true, true, true, RAG, true, PAGED>(a, i - n_update, &pa);
}

// The pass's grid is num_splits x Hkv x B workgroups whether or not seq_lens is given (B is 1 then),
// or pass_budget + Hkv x B for the balanced partition (the list of a (b, KV head) is cut into
// num_splits slices as in the unragged pass); a ragged batch (RAG): (num_splits + B) x Hkv, the
// ragged pass's grid.
template <int D, int G, bool PAGED, bool RAG = false>
hipError_t launch_planned_p(const AttnP& a, const kvskip_plan_args& pa, const kvskip_update_args* u, hipStream_t s) {
  const dim3 blk(NT);
  const int nslot = pa.slot_count > 0 ? pa.slot_count : a.num_splits;
  const int n_pass = RAG ? static_cast<int>(attn_grid(a).x)
                         : (pa.pass_budget > 0 ? pa.pass_budget + a.Hkv * a.B : nslot * a.Hkv * a.B);
  if (u == nullptr) {
    hipLaunchKernelGGL((planned_split_kernel<D, G, 0, PAGED, RAG>), dim3(n_pass), blk, 0, s, a, pa,
                       kvskip_update_args{});
    return hipGetLastError();
  }
  const int nb = (u->T + BLK - 1) / BLK;
  const dim3 grid(n_pass + u->B * u->Hkv);
  if (nb <= 2 * WAVE) hipLaunchKernelGGL((planned_split_kernel<D, G, 2, PAGED, RAG>), grid, blk, 0, s, a, pa, *u);
  else if (nb <= 4 * WAVE) hipLaunchKernelGGL((planned_split_kernel<D, G, 4, PAGED, RAG>), grid, blk, 0, s, a, pa, *u);
  else if (nb <= 8 * WAVE) hipLaunchKernelGGL((planned_split_kernel<D, G, 8, PAGED, RAG>), grid, blk, 0, s, a, pa, *u);
  else if (nb <= 16 * WAVE) hipLaunchKernelGGL((planned_split_kernel<D, G, 16, PAGED, RAG>), grid, blk, 0, s, a, pa, *u);
  else hipLaunchKernelGGL((planned_split_kernel<D, G, CARRY_MAX_R, PAGED, RAG>), grid, blk, 0, s, a, pa, *u);
  return hipGetLastError();
}


}  // namespace
}  // namespace kvs
