// Block selection on the device: the GQA-union rules of kernels/kvskip.py:130-147 ("tau", "topp")
// over per-block statistics, the kept-first block list of make_plan (kernels/kvskip.py:79-85) and the
// per-block scales of the two-pass V-skip's second pass (kernels/kvskip.py:169-172). select_core is
// shared by the selection's own kernel (select.hip) and by the second pass with the selection in its
// prologue (attn_vskip.hip).
#pragma once
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

// Selection of (KV head h, sequence b) by the first SW wavefronts of a workgroup: each wavefront
// takes query heads g = wave + 4 j; lane holds blocks i = lane + 64 r (r < R, nb <= 64 R). A head
// keeps its blocks by the rule, the group keeps the union plus block 0 and the `local` newest. Leaves
// the kept mask in sKeep[R] (LDS; bit i % 64 of slot i / 64) and, if sLk is given, each query head's
// log-sum-exp over its kept blocks in sLk[g] (+inf where they hold no mass, so that exp(blk_max - sLk)
// is that head's scale, as written below); with `write`, the outputs of kvskip_select: the keep mask,
// the list (kept ascending, then the others ascending, as a stable sort of ~keep) and each head's
// scale exp(blk_max - lse_kept). Ends with the workgroup's barrier after sKeep / sLk are written.
template <int R>
__device__ void select_core(const kvskip_select_args& a, int h, int b, uint64_t* sKeep, float* sLk, bool write) {
  constexpr int HPW = (SEL_MAX_G + SW - 1) / SW;  // query heads per wavefront at most
  const int G = a.Hq / a.Hkv;
  const int nb = a.nb;
  const int tid = threadIdx.x, lane = tid % WAVE;
  const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE);
  const int64_t bh = static_cast<int64_t>(b) * a.Hkv + h;
  const int64_t hrow0 = static_cast<int64_t>(b) * a.Hq + static_cast<int64_t>(h) * G;
  __shared__ uint64_t sKm[SEL_MAX_G][R];  // per query head: the blocks its rule keeps
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

  if (write && a.keep != nullptr)
    for (int i = tid; i < nb; i += SW * WAVE) a.keep[bh * nb + i] = (kn[i / WAVE] >> (i % WAVE)) & 1;

  if (write && a.block_idx != nullptr) {  // wavefront w writes slots r = w + SW t; positions from the slots before
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

  const bool scales = write && a.blk_scale != nullptr;
  if (scales || sLk != nullptr) {
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
      if (sLk != nullptr && lane == 0) sLk[g] = sum > 0.f ? lk : __builtin_inff();
      if (scales) {
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
  __syncthreads();
}

}  // namespace
}  // namespace kvs
