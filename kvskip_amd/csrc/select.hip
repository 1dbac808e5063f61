// Block selection on the device: the GQA-union rules of kernels/kvskip.py:130-147 ("tau", "topp")
// over per-block statistics, the kept-first block list of make_plan (kernels/kvskip.py:79-85) and the
// per-block scales of the two-pass V-skip's second pass (kernels/kvskip.py:169-172), so that the
// two-pass V-skip runs pass 1 -> select -> pass 2 with no host work in between.
#include "planner_common.hpp"

namespace kvs {
namespace {

constexpr int SW = 4;       // wavefronts per selection workgroup
constexpr int SEL_MAX_G = 8;

// A head's statistics of the blocks lane + 64 r (r < RU, clamped into [0, nb)): every load issued
// before any is used, so the wavefront waits for one memory round trip, not one per slot.
template <int R>
__device__ __forceinline__ void load_stats(const float* bm, const float* bs, int nb, int RU, int lane, float (&m)[R],
                                           float (&s)[R]) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int ic = min(lane + WAVE * r, nb - 1);
    m[r] = r < RU ? bm[ic] : NEG_INF;
    s[r] = r < RU ? bs[ic] : 0.f;
  }
}

// Block log-weight blk_max + log blk_sum (-inf where the block holds nothing or is past nb).
__device__ __forceinline__ float log_weight(float m, float s, bool in) { return in && s > 0.f ? m + __logf(s) : NEG_INF; }

// Workgroup (KV head h, sequence b): each wavefront takes query heads g = wave + 4 j; lane holds
// blocks i = lane + 64 r (r < R, nb <= 64 R). A head keeps its blocks by the rule, the group keeps
// the union plus block 0 and the `local` newest; then the kept mask, the list (kept ascending, then
// the others ascending, as a stable sort of ~keep) and each head's scale exp(blk_max - lse_kept).
template <int R>
__global__ void __launch_bounds__(SW * WAVE) select_kernel(const kvskip_select_args a) {
  constexpr int HPW = (SEL_MAX_G + SW - 1) / SW;  // query heads per wavefront at most
  const int h = blockIdx.x, b = blockIdx.y;
  const int G = a.Hq / a.Hkv;
  const int nb = a.nb;
  const int tid = threadIdx.x, lane = tid % WAVE;
  const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE);
  const int64_t bh = static_cast<int64_t>(b) * a.Hkv + h;
  const int64_t hrow0 = static_cast<int64_t>(b) * a.Hq + static_cast<int64_t>(h) * G;
  __shared__ uint64_t sKm[SEL_MAX_G][R];  // per query head: the blocks its rule keeps
  __shared__ uint64_t sKeep[R];           // the group's union with sink and local blocks
  __shared__ uint64_t sHist[SW][256];     // each wavefront's top-p histogram
  // slots past the last block's group of 4 hold nothing (uniform)
  const int RU = R <= 4 ? R : min(R, 4 * ((nb + 4 * WAVE - 1) / (4 * WAVE)));
  // a head's statistics stay in registers for its scales when they fit (else they are loaded again)
  constexpr bool KEEP_REGS = R <= 16;
  float bmk[KEEP_REGS ? HPW : 1][KEEP_REGS ? R : 1], xk[KEEP_REGS ? HPW : 1][KEEP_REGS ? R : 1];

#pragma unroll
  for (int j = 0; j < HPW; ++j) {
    const int g = wave + SW * j;
    if (g >= G) break;
    float x[R], bmv[R];
    {
      float bsv[R];
      load_stats<R>(a.blk_max + (hrow0 + g) * nb, a.blk_sum + (hrow0 + g) * nb, nb, RU, lane, bmv, bsv);
#pragma unroll
      for (int r = 0; r < R; ++r) x[r] = log_weight(bmv[r], bsv[r], r < RU && lane + WAVE * r < nb);
    }
    if constexpr (KEEP_REGS) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        bmk[j][r] = bmv[r];
        xk[j][r] = x[r];
      }
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
      const uint32_t theta = any ? topp_theta<R>(key, w, RU, a.value, mx - lse, sHist[wave]) : 0xffffffffu;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint64_t m = __ballot(any && lane + WAVE * r < nb && x[r] != NEG_INF && key[r] >= theta);
        if (lane == 0) sKm[g][r] = m;
      }
    }
  }
  __syncthreads();
  if (tid < R) {  // thread r: slot r's union over the group, the sink and the local blocks
    uint64_t u = 0;
#pragma unroll
    for (int g = 0; g < SEL_MAX_G; ++g)
      if (g < G) u |= sKm[g][tid];
    const int i0 = WAVE * tid;  // blocks i0 .. i0 + 63 of this slot
    const int n_in = min(max(nb - i0, 0), WAVE);
    const uint64_t valid = n_in == WAVE ? ~0ull : ((1ull << n_in) - 1);
    const int a0 = max(nb - a.local, 0) - i0;  // slot bits >= a0 are local blocks
    const uint64_t local = a0 <= 0 ? ~0ull : (a0 >= WAVE ? 0ull : ~((1ull << a0) - 1));
    sKeep[tid] = (u | local | (tid == 0 ? 1ull : 0ull)) & valid;
  }
  __syncthreads();
  const uint64_t* kn = sKeep;

  if (a.keep != nullptr)
    for (int i = tid; i < nb; i += SW * WAVE) a.keep[bh * nb + i] = (kn[i / WAVE] >> (i % WAVE)) & 1;

  if (a.block_idx != nullptr) {  // wavefront w writes slots r = w + SW t; positions from the slots before
    int total = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) total += __popcll(kn[r]);
    const uint64_t below = (1ull << lane) - 1;  // lanes before this one
    int base_k = 0, base_u = total;
    int32_t* bi = a.block_idx + bh * nb;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int n_valid = min(max(nb - WAVE * r, 0), WAVE);
      const uint64_t valid = n_valid == WAVE ? ~0ull : ((1ull << n_valid) - 1);
      if (r % SW == wave) {
        const int i = lane + WAVE * r;
        const bool k = (kn[r] >> lane) & 1;
        if (i < nb) bi[k ? base_k + __popcll(kn[r] & below) : base_u + __popcll(valid & ~kn[r] & below)] = i;
      }
      base_k += __popcll(kn[r]);
      base_u += __popcll(valid & ~kn[r]);
    }
    if (tid == 0) a.block_cnt[bh] = total;
  }

  if (a.blk_scale != nullptr) {
#pragma unroll
    for (int j = 0; j < HPW; ++j) {
      const int g = wave + SW * j;
      if (g >= G) break;
      float bmv[R], x[R];
      if constexpr (KEEP_REGS) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          bmv[r] = bmk[j][r];
          x[r] = xk[j][r];
        }
      } else {
        float bsv[R];
        load_stats<R>(a.blk_max + (hrow0 + g) * nb, a.blk_sum + (hrow0 + g) * nb, nb, RU, lane, bmv, bsv);
#pragma unroll
        for (int r = 0; r < R; ++r) x[r] = log_weight(bmv[r], bsv[r], r < RU && lane + WAVE * r < nb);
      }
      // log-sum-exp over the kept blocks: the max first, then the scaled sum (independent terms)
      float m = NEG_INF;
#pragma unroll
      for (int r = 0; r < R; ++r)
        if ((kn[r] >> lane) & 1) m = fmaxf(m, x[r]);
      m = wave_max(m);
      float sum = 0.f;
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (((kn[r] >> lane) & 1) && x[r] != NEG_INF) sum += __expf(x[r] - m);
      sum = wave_sum(sum);
      const float lk = sum > 0.f ? m + __logf(sum) : 0.f;
      float* sc = a.blk_scale + bh * nb * G + g;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int i = lane + WAVE * r;
        const bool kept = (kn[r] >> lane) & 1;
        if (i < nb) sc[static_cast<int64_t>(i) * G] = (sum > 0.f && kept) ? __expf(bmv[r] - lk) : 0.f;
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
