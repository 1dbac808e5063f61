// Block selection on the device: the GQA-union rules of kernels/kvskip.py:130-147 ("tau", "topp")
// over per-block statistics, the kept-first block list of make_plan (kernels/kvskip.py:79-85) and the
// per-block scales of the two-pass V-skip's second pass (kernels/kvskip.py:169-172), so that the
// two-pass V-skip runs pass 1 -> select -> pass 2 with no host work in between.
#include "planner_common.hpp"

namespace kvs {
namespace {

constexpr int SW = 4;       // wavefronts per selection workgroup
constexpr int SEL_MAX_G = 8;

// Block i's log-weight blk_max + log blk_sum (-inf where the block holds nothing).
__device__ __forceinline__ float log_weight(const float* bm, const float* bs, int i) {
  const float s = bs[i];
  return s > 0.f ? bm[i] + __logf(s) : NEG_INF;
}

// Workgroup (KV head h, sequence b): each wavefront takes query heads g = wave + 4 j; lane holds
// blocks i = lane + 64 r (r < R, nb <= 64 R). A head keeps its blocks by the rule, the group keeps
// the union plus block 0 and the `local` newest; then the kept mask, the list (kept ascending, then
// the others ascending, as a stable sort of ~keep) and each head's scale exp(blk_max - lse_kept).
template <int R>
__global__ void __launch_bounds__(SW * WAVE) select_kernel(const kvskip_select_args a) {
  const int h = blockIdx.x, b = blockIdx.y;
  const int G = a.Hq / a.Hkv;
  const int nb = a.nb;
  const int tid = threadIdx.x, lane = tid % WAVE;
  const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE);
  const int64_t bh = static_cast<int64_t>(b) * a.Hkv + h;
  const int64_t hrow0 = static_cast<int64_t>(b) * a.Hq + static_cast<int64_t>(h) * G;
  __shared__ uint64_t sKm[SEL_MAX_G][R];  // per query head: the blocks its rule keeps
  __shared__ uint64_t sKeep[R];           // the group's union with sink and local blocks
  // slots past the last block's group of 4 hold nothing (uniform)
  const int RU = R <= 4 ? R : min(R, 4 * ((nb + 4 * WAVE - 1) / (4 * WAVE)));

  for (int g = wave; g < G; g += SW) {
    const float* bm = a.blk_max + (hrow0 + g) * nb;
    const float* bs = a.blk_sum + (hrow0 + g) * nb;
    float x[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int i = lane + WAVE * r;
      x[r] = (r < RU && i < nb) ? log_weight(bm, bs, i) : NEG_INF;
    }
    float mx = NEG_INF;
#pragma unroll
    for (int r = 0; r < R; ++r) mx = fmaxf(mx, x[r]);
    mx = wave_max(mx);
    float se = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (r < RU && x[r] != NEG_INF) se += __expf(x[r] - mx);
    const float tot = wave_sum(se);
    const bool any = tot > 0.f;                // a head with no mass keeps nothing by its rule
    const float lse = any ? mx + __logf(tot) : 0.f;
    float w[R];
    uint32_t key[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float y = x[r] - lse;
      w[r] = (r < RU && x[r] != NEG_INF) ? __expf(y) : 0.f;
      key[r] = x[r] != NEG_INF ? fkey(y) : 0u;
    }
    if (a.rule == 0) {  // tau: weight >= value
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint64_t m = __ballot(any && lane + WAVE * r < nb && x[r] != NEG_INF && w[r] >= a.value);
        if (lane == 0) sKm[g][r] = m;
      }
    } else {            // topp: the fewest blocks reaching value
      const uint32_t theta = any ? topp_theta<R>(key, w, RU, a.value) : 0xffffffffu;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint64_t m = __ballot(any && lane + WAVE * r < nb && x[r] != NEG_INF && key[r] >= theta);
        if (lane == 0) sKm[g][r] = m;
      }
    }
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      uint64_t u = 0;
      for (int g = 0; g < G; ++g) u |= sKm[g][r];
      const int i = lane + WAVE * r;
      const bool k = i < nb && (((u >> lane) & 1) || always_block(i, nb, a.local));
      const uint64_t m = __ballot(k);
      if (lane == 0) sKeep[r] = m;
    }
  }
  __syncthreads();
  const uint64_t* kn = sKeep;

  if (a.keep != nullptr)
    for (int i = tid; i < nb; i += SW * WAVE) a.keep[bh * nb + i] = (kn[i / WAVE] >> (i % WAVE)) & 1;

  if (a.block_idx != nullptr && wave == 0) {
    int total = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) total += __popcll(kn[r]);
    const uint64_t below = (1ull << lane) - 1;  // lanes before this one
    int base_k = 0, base_u = total;
    int32_t* bi = a.block_idx + bh * nb;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int i = lane + WAVE * r;
      const int n_valid = min(max(nb - WAVE * r, 0), WAVE);
      const uint64_t valid = n_valid == WAVE ? ~0ull : ((1ull << n_valid) - 1);
      const bool k = (kn[r] >> lane) & 1;
      if (i < nb) {
        const int pos = k ? base_k + __popcll(kn[r] & below) : base_u + __popcll(valid & ~kn[r] & below);
        bi[pos] = i;
      }
      base_k += __popcll(kn[r]);
      base_u += __popcll(valid & ~kn[r]);
    }
    if (lane == 0) a.block_cnt[bh] = total;
  }

  if (a.blk_scale != nullptr) {
    for (int g = wave; g < G; g += SW) {
      const float* bm = a.blk_max + (hrow0 + g) * nb;
      const float* bs = a.blk_sum + (hrow0 + g) * nb;
      float m = NEG_INF, s = 0.f;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int i = lane + WAVE * r;
        if (r < RU && i < nb && ((kn[r] >> lane) & 1)) lse_push(m, s, log_weight(bm, bs, i));
      }
      lse_wave(m, s);
      const float lk = s > 0.f ? m + __logf(s) : 0.f;
      float* sc = a.blk_scale + bh * nb * G + g;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int i = lane + WAVE * r;
        if (i < nb) sc[static_cast<int64_t>(i) * G] = (s > 0.f && ((kn[r] >> lane) & 1)) ? __expf(bm[i] - lk) : 0.f;
      }
    }
  }
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
