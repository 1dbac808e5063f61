// Block selection on the device: the GQA-union rules of kernels/kvskip.py:130-147 ("tau", "topp")
// over per-block statistics, the kept-first block list of make_plan (kernels/kvskip.py:79-85) and the
// per-block scales of the two-pass V-skip's second pass (kernels/kvskip.py:169-172), so that the
// two-pass V-skip runs pass 1 -> select -> pass 2 with no host work in between.
#include "select.hpp"

namespace kvs {
namespace {

template <int R>
__global__ void __launch_bounds__(SW * WAVE) select_kernel(const kvskip_select_args a) {
  __shared__ uint64_t sKeep[R];  // the group's union with sink and local blocks
  select_core<R>(a, blockIdx.x, blockIdx.y, sKeep, nullptr, true);
}

// One wavefront per (b, KV head): the kept-first list of a keep mask (u8, nonzero = kept).
__global__ void __launch_bounds__(WAVE) block_list_kernel(const uint8_t* keep, int nb, int32_t* block_idx,
                                                          int32_t* block_cnt) {
  const int64_t bh = blockIdx.x;
  const int lane = threadIdx.x;
  const uint8_t* kp = keep + bh * nb;
  int32_t* bi = block_idx + bh * nb;
  const uint64_t below = (1ull << lane) - 1;
  int total = 0;
  for (int c = 0; c < nb; c += WAVE) total += __popcll(__ballot(c + lane < nb && kp[c + lane] != 0));
  int base_k = 0, base_u = total;
  for (int c = 0; c < nb; c += WAVE) {
    const int i = c + lane;
    const bool in = i < nb;
    const bool k = in && kp[i] != 0;
    const uint64_t mk = __ballot(k), mu = __ballot(in && !k);
    if (in) bi[k ? base_k + __popcll(mk & below) : base_u + __popcll(mu & below)] = i;
    base_k += __popcll(mk);
    base_u += __popcll(mu);
  }
  if (lane == 0) block_cnt[bh] = total;
}

}  // namespace

hipError_t launch_select(const kvskip_select_args& a, hipStream_t s) {
  const dim3 grid(a.Hkv, a.B), block(SW * WAVE);
  const int r = (a.nb + WAVE - 1) / WAVE;
  if (r <= 1) hipLaunchKernelGGL(select_kernel<1>, grid, block, 0, s, a);
  else if (r <= 2) hipLaunchKernelGGL(select_kernel<2>, grid, block, 0, s, a);
  else if (r <= 4) hipLaunchKernelGGL(select_kernel<4>, grid, block, 0, s, a);
  else if (r <= 8) hipLaunchKernelGGL(select_kernel<8>, grid, block, 0, s, a);
  else if (r <= 16) hipLaunchKernelGGL(select_kernel<16>, grid, block, 0, s, a);
  else if (r <= 32) hipLaunchKernelGGL(select_kernel<32>, grid, block, 0, s, a);
  else hipLaunchKernelGGL(select_kernel<64>, grid, block, 0, s, a);
  return hipGetLastError();
}

hipError_t launch_block_list(const uint8_t* keep, int B, int Hkv, int nb, int32_t* block_idx, int32_t* block_cnt,
                             hipStream_t s) {
  hipLaunchKernelGGL(block_list_kernel, dim3(B * Hkv), dim3(WAVE), 0, s, keep, nb, block_idx, block_cnt);
  return hipGetLastError();
}

}  // namespace kvs
