// Device-side refresh planner for gfx950: plan (before the attention pass) and update (after
// it), plus the two helpers that let the whole loop start on the device: per-block key sums
// of a prefix and the token index of a decode step.
//
// Policy (one KV head = one group of G query heads; blocks of 64 tokens): a head attends its
// stored set + block 0 + the `local` newest blocks. Before the pass, plan estimates the mass
// outside that set from the block log-sum-exps recorded at the head's last refresh, moved by
// how far each block's centroid score q.c_b has drifted since (est_b = lse_ref_b + cs_b -
// cs_ref_b), against the previous step's attended log-sum-exp; if the estimate (optionally
// calibrated) exceeds delta, or the set is max_age steps old, or the head is flagged, the
// head refreshes: it reads every block this step, and update rebuilds its set from the block
// statistics of that same pass (each query head's top-p blocks, union over the group).
//
// plan:   workgroup of 4 wavefronts per (b, KV head). Centroid scores with 16 lanes per block
//         row (fp32 key sums, 4 block rows per wavefront step); the drift estimate is folded
//         into the same pass (lane 16 r + g keeps head g's running log-sum-exp), so no LDS
//         copy of the scores is needed; the block list is compacted in ascending order by
//         wavefront ballots.
// update: one wavefront per query head of the group (G wavefronts). Top-p by an exact
//         bitwise search for the largest score key whose upper set holds >= level of the mass
//         (the fewest blocks reaching level; ties at the threshold are all kept).
#include "common.hpp"
#include "internal.hpp"

namespace kvs {
namespace {

__device__ __forceinline__ bool always_block(int blk, int nb, int local) { return blk == 0 || blk >= nb - local; }

__device__ __forceinline__ float clamped_logit(float x) {
  x = fminf(fmaxf(x, 1e-6f), 1.f - 1e-6f);
  return __logf(x) - __logf(1.f - x);
}

// Merge (m, s) log-sum-exp pairs: (m1, s1) <- (m1, s1) + (m2, s2).
__device__ __forceinline__ void lse_merge(float& m1, float& s1, float m2, float s2) {
  if (s2 <= 0.f) return;
  if (s1 <= 0.f) {
    m1 = m2;
    s1 = s2;
    return;
  }
  if (m2 > m1) {
    s1 = s1 * __expf(m1 - m2) + s2;
    m1 = m2;
  } else {
    s1 += s2 * __expf(m2 - m1);
  }
}

// Wavefront merge of (m, s) pairs over the lanes selected by xor masks 16 and 32.
__device__ __forceinline__ void lse_merge_rows(float& m, float& s) {
#pragma unroll
  for (int o = 16; o < WAVE; o <<= 1) {
    const float m2 = __shfl_xor(m, o, WAVE), s2 = __shfl_xor(s, o, WAVE);
    lse_merge(m, s, m2, s2);
  }
}
__device__ __forceinline__ void lse_merge_wave(float& m, float& s) {
#pragma unroll
  for (int o = 1; o < WAVE; o <<= 1) {
    const float m2 = __shfl_xor(m, o, WAVE), s2 = __shfl_xor(s, o, WAVE);
    lse_merge(m, s, m2, s2);
  }
}

// Ascending compaction of {blk < nb : pred(blk)} into out[], by one wavefront; returns the count.
template <typename Pred>
__device__ __forceinline__ int compact_wave(int nb, int lane, int* out, Pred pred) {
  int base = 0;
  for (int c0 = 0; c0 < nb; c0 += WAVE) {
    const int blk = c0 + lane;
    const bool f = blk < nb && pred(blk);
    const uint64_t mask = __ballot(f);
    const int off = __popcll(mask & ((uint64_t(1) << lane) - 1));
    if (f) out[base + off] = blk;
    base += __popcll(mask);
  }
  return base;
}

constexpr int PNT = 256;  // plan workgroup

template <int D, int G>
__global__ void __launch_bounds__(PNT) plan_kernel(const kvskip_plan_args p) {
  constexpr int DL = D / 16;  // dims per lane in the centroid pass
  const int h = blockIdx.x, b = blockIdx.y;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE;
  const int nb = (p.T + BLK - 1) / BLK;
  const int64_t bh = static_cast<int64_t>(b) * p.Hkv + h;
  const int64_t row0 = (static_cast<int64_t>(b) * p.Hq + static_cast<int64_t>(h) * G) * p.NBC;  // head g: + g*NBC
  float* csum = p.csum + bh * p.NBC * D;
  const uint8_t* keep = p.keep + bh * p.NBC;
  int* bi = p.block_idx + bh * p.NBC;
  const int fl = p.flags[h];
  __shared__ float sM[PNT / WAVE][G], sS[PNT / WAVE][G];
  __shared__ int sTrig;

  if (fl & 2) {  // token-index head: index blocks + sink + local, never refreshes
    const uint8_t* idx = p.idx != nullptr ? p.idx + static_cast<int64_t>(b) * p.NBC : nullptr;
    if (wave == 0) {
      const int cnt = compact_wave(nb, lane, bi, [&](int i) { return (idx != nullptr && idx[i] != 0) || always_block(i, nb, p.local); });
      if (lane == 0) {
        p.block_cnt[bh] = cnt;
        p.trig[bh] = 0;
      }
    }
    return;
  }
  const bool uni = p.idx != nullptr && ((fl & 4) || (p.aix != nullptr && p.aix[bh] != 0));
  const uint8_t* idx = uni ? p.idx + static_cast<int64_t>(b) * p.NBC : nullptr;
  auto attended = [&](int i) { return keep[i] != 0 || always_block(i, nb, p.local) || (uni && idx[i] != 0); };

  if (p.add_token && tid < D) {  // the key appended by this step joins its block's sum
    const int t = p.T - 1;
    const uint16_t* kr = reinterpret_cast<const uint16_t*>(p.k) + b * p.k_sb + h * p.k_sh +
                         static_cast<int64_t>(t) * p.k_st;
    csum[static_cast<int64_t>(t / BLK) * D + tid] += __uint_as_float(static_cast<uint32_t>(kr[tid]) << 16);
  }
  __syncthreads();

  // Centroid scores + drift estimate. Lane (rs = lane/16, c16 = lane%16): block row rs of
  // each step, dims {4*c16 + j, 64 + 4*c16 + j} (D = 128) or {4*c16 + j} (D = 64).
  const int rs = lane >> 4, c16 = lane & 15;
  float qf[G][DL];
  {
    const uint16_t* q = reinterpret_cast<const uint16_t*>(p.q);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const uint16_t* qp = q + b * p.q_sb + (static_cast<int64_t>(h) * G + g) * p.q_sh;
#pragma unroll
      for (int u = 0; u < DL / 4; ++u)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          qf[g][4 * u + j] = __uint_as_float(static_cast<uint32_t>(qp[64 * u + 4 * c16 + j]) << 16) * p.scale;
    }
  }
  float em = NEG_INF, es = 0.f;  // head g = c16 (if < G): running log-sum-exp of est over unattended blocks
  for (int base = 4 * wave; base < nb; base += 4 * (PNT / WAVE)) {
    const int blk = base + rs;
    const bool ok = blk < nb;
    float cv[DL];
    if (ok) {
      const float* cp = csum + static_cast<int64_t>(blk) * D;
#pragma unroll
      for (int u = 0; u < DL / 4; ++u) {
        const float4 t = *reinterpret_cast<const float4*>(cp + 64 * u + 4 * c16);
        cv[4 * u] = t.x;
        cv[4 * u + 1] = t.y;
        cv[4 * u + 2] = t.z;
        cv[4 * u + 3] = t.w;
      }
    } else {
#pragma unroll
      for (int j = 0; j < DL; ++j) cv[j] = 0.f;
    }
    const float inv_n = 1.f / static_cast<float>(blk == nb - 1 ? p.T - blk * BLK : BLK);
    float mine = 0.f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float d = 0.f;
#pragma unroll
      for (int j = 0; j < DL; ++j) d = fmaf(qf[g][j], cv[j], d);
      d += dpp<DPP_XOR1>(d);
      d += dpp<DPP_XOR2>(d);
      d += dpp<DPP_HALF_MIRROR>(d);
      d += dpp<DPP_MIRROR>(d);
      if (c16 == g) mine = d * inv_n;
    }
    if (ok && c16 < G) {
      p.cs_now[row0 + static_cast<int64_t>(c16) * p.NBC + blk] = mine;
      if (!attended(blk)) {
        const int64_t r = row0 + static_cast<int64_t>(c16) * p.NBC + blk;
        lse_push(em, es, p.lse_ref[r] + mine - p.cs_ref[r]);
      }
    }
  }
  lse_merge_rows(em, es);
  if (rs == 0 && c16 < G) {
    sM[wave][c16] = em;
    sS[wave][c16] = es;
  }
  __syncthreads();

  if (tid == 0) {
    float miss = 0.f;
    for (int g = 0; g < G; ++g) {
      float M = NEG_INF, S = 0.f;
      for (int w = 0; w < PNT / WAVE; ++w) lse_merge(M, S, sM[w][g], sS[w][g]);
      if (S > 0.f) {
        const float est = M + __logf(S);
        const float la = p.lse_att[static_cast<int64_t>(b) * p.Hq + static_cast<int64_t>(h) * G + g];
        miss = fmaxf(miss, 1.f / (1.f + __expf(la - est)));
      }
    }
    if (p.est != nullptr) p.est[bh] = miss;
    float dec = miss;
    if (p.calib != nullptr && p.calib_on)
      dec = p.calib_kind ? miss + p.calib[bh] : 1.f / (1.f + __expf(-(clamped_logit(miss) + p.calib[bh])));
    const int a = p.age[bh] + 1;
    const bool tr = dec > p.delta || a >= p.max_age || (fl & 1);
    p.age[bh] = tr ? 0 : a;
    p.trig[bh] = tr ? 1 : 0;
    sTrig = tr;
  }
  __syncthreads();

  if (wave == 0) {
    const bool tr = sTrig != 0;
    const int cnt = compact_wave(nb, lane, bi, [&](int i) { return tr || attended(i); });
    if (lane == 0) p.block_cnt[bh] = cnt;
  }
}

template <int G>
__global__ void update_kernel(const kvskip_update_args p) {
  extern __shared__ float smem[];
  const int h = blockIdx.x, b = blockIdx.y;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE;  // wave = query head g
  const int nb = (p.T + BLK - 1) / BLK;
  const int64_t bh = static_cast<int64_t>(b) * p.Hkv + h;
  const int64_t hrow = static_cast<int64_t>(b) * p.Hq + static_cast<int64_t>(h) * G + wave;
  float* x = smem + static_cast<int64_t>(wave) * nb;                           // [G][nb] block log-weights
  uint8_t* skeep = reinterpret_cast<uint8_t*>(smem + static_cast<int64_t>(G) * nb);  // [nb]
  __shared__ float sReal[G];
  uint8_t* keep = p.keep + bh * p.NBC;
  const bool tr = p.trig[bh] != 0;
  const int fl = p.flags != nullptr ? p.flags[h] : 0;

  float mx = NEG_INF;
  for (int i = lane; i < nb; i += WAVE) {
    const float v = p.blk_max[hrow * nb + i] + __logf(p.blk_sum[hrow * nb + i]);  // -inf where not read
    x[i] = v;
    mx = fmaxf(mx, v);
  }
  for (int i = tid; i < nb; i += G * WAVE) skeep[i] = 0;
  mx = wave_max(mx);
  __syncthreads();

  if (tr && p.calib != nullptr) {  // the mass the attended set missed (this head read every block)
    const bool uni = p.idx != nullptr && ((fl & 4) || (p.aix != nullptr && p.aix[bh] != 0));
    const uint8_t* idx = uni ? p.idx + static_cast<int64_t>(b) * p.NBC : nullptr;
    float mi = NEG_INF, si = 0.f, mo = NEG_INF, so = 0.f;
    for (int i = lane; i < nb; i += WAVE) {
      if (keep[i] != 0 || always_block(i, nb, p.local) || (uni && idx[i] != 0))
        lse_push(mi, si, x[i]);
      else
        lse_push(mo, so, x[i]);
    }
    lse_merge_wave(mi, si);
    lse_merge_wave(mo, so);
    if (lane == 0) sReal[wave] = so > 0.f ? 1.f / (1.f + __expf((mi + __logf(si)) - (mo + __logf(so)))) : 0.f;
  }
  if (tr) {
    float se = 0.f;
    for (int i = lane; i < nb; i += WAVE) se += __expf(x[i] - mx);
    const float lse = mx + __logf(wave_sum(se));
    // Largest key theta (order-preserving bits of y = x - lse) whose upper set {key >= theta}
    // holds >= level of the mass; keep exactly that upper set.
    auto key_of = [](float y) -> uint32_t {
      const uint32_t u = __float_as_uint(y);
      return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    };
    uint32_t theta = 0;
    for (int bit = 31; bit >= 0; --bit) {
      const uint32_t cand = theta | (1u << bit);
      float acc = 0.f;
      for (int i = lane; i < nb; i += WAVE) {
        const float y = x[i] - lse;
        if (key_of(y) >= cand) acc += __expf(y);
      }
      if (wave_sum(acc) >= p.level) theta = cand;
    }
    for (int i = lane; i < nb; i += WAVE)
      if (key_of(x[i] - lse) >= theta) skeep[i] = 1;
    for (int i = lane; i < p.NBC; i += WAVE) {
      p.lse_ref[hrow * p.NBC + i] = i < nb ? x[i] : NEG_INF;
      p.cs_ref[hrow * p.NBC + i] = i < nb ? p.cs_now[hrow * p.NBC + i] : 0.f;
    }
  }
  __syncthreads();
  if (tr && p.calib != nullptr && tid == 0) {
    float real = 0.f;
    for (int g = 0; g < G; ++g) real = fmaxf(real, sReal[g]);
    const float est = p.est[bh];
    const float resid = p.calib_kind ? real - est : clamped_logit(real) - clamped_logit(est);
    float c = p.calib_kind == 2 ? fmaxf((1.f - p.calib_rate) * p.calib[bh], resid)
                                : (1.f - p.calib_rate) * p.calib[bh] + p.calib_rate * resid;
    if (!p.calib_free) c = fmaxf(c, 0.f);
    p.calib[bh] = c;
    if (p.aix != nullptr && c > p.aix_thr) p.aix[bh] = 1;
  }
  if (tr) {
    for (int i = tid; i < p.NBC; i += G * WAVE)
      keep[i] = (i < nb && (skeep[i] != 0 || always_block(i, nb, p.local))) ? 1 : 0;
  }
  // Attended log-sum-exp for the next step (every head), over the (new) stored set + always.
  float m2 = NEG_INF, s2 = 0.f;
  for (int i = lane; i < nb; i += WAVE) {
    const bool k = tr ? (skeep[i] != 0) : (keep[i] != 0);
    if (k || always_block(i, nb, p.local)) lse_push(m2, s2, x[i]);
  }
  lse_merge_wave(m2, s2);
  if (lane == 0) p.lse_att[hrow] = s2 > 0.f ? m2 + __logf(s2) : NEG_INF;
}

// csum[b, h, blk, d] = sum over the block's rows t < T of k[b, h, t, d]; zero for blk >= nb.
template <int D>
__global__ void __launch_bounds__(D) block_sums_kernel(const uint16_t* k, int64_t k_sb, int64_t k_sh, int64_t k_st,
                                                       int Hkv, int T, float* csum, int NBC) {
  const int blk = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int d = threadIdx.x;
  const int t0 = blk * BLK, t1 = min(T, t0 + BLK);
  const uint16_t* kb = k + b * k_sb + h * k_sh + d;
  float a = 0.f;
  for (int t = t0; t < t1; ++t) a += __uint_as_float(static_cast<uint32_t>(kb[static_cast<int64_t>(t) * k_st]) << 16);
  csum[((static_cast<int64_t>(b) * Hkv + h) * NBC + blk) * D + d] = a;
}

// idx[b, blk] = any position j < T of the block with ids[j] == cur (j < T-1) or ids[j-1] == cur
// (j-1 < T-1), cur = ids[T-1]. One wavefront per block, lane = token.
__global__ void __launch_bounds__(256) token_index_kernel(const int32_t* ids, int64_t stride, int T, uint8_t* idx,
                                                          int NBC) {
  const int b = blockIdx.y;
  const int blk = blockIdx.x * 4 + threadIdx.x / WAVE;
  const int lane = threadIdx.x % WAVE;
  if (blk >= NBC) return;
  const int32_t* x = ids + b * stride;
  const int32_t cur = x[T - 1];
  const int j = blk * BLK + lane;
  bool hit = false;
  if (j < T) {
    const bool same = j < T - 1 && x[j] == cur;
    const bool after = j >= 1 && j - 1 < T - 1 && x[j - 1] == cur;
    hit = same || after;
  }
  const uint64_t m = __ballot(hit);
  if (lane == 0) idx[static_cast<int64_t>(b) * NBC + blk] = m != 0 ? 1 : 0;
}

template <int D, int G>
hipError_t launch_plan_t(const kvskip_plan_args& p, hipStream_t s) {
  hipLaunchKernelGGL((plan_kernel<D, G>), dim3(p.Hkv, p.B), dim3(PNT), 0, s, p);
  return hipGetLastError();
}

template <int G>
hipError_t launch_update_t(const kvskip_update_args& p, hipStream_t s) {
  const int nb = (p.T + BLK - 1) / BLK;
  const size_t smem = static_cast<size_t>(G) * nb * sizeof(float) + nb;
  hipLaunchKernelGGL((update_kernel<G>), dim3(p.Hkv, p.B), dim3(G * WAVE), smem, s, p);
  return hipGetLastError();
}

}  // namespace

// LDS of update: G * nb floats + nb bytes, within 64 KiB.
int planner_max_blocks(int G) { return (64 * 1024) / (4 * G + 1); }

hipError_t launch_plan(const kvskip_plan_args& p, hipStream_t s) {
  const int G = p.Hq / p.Hkv;
#define KVS_CASE(DD, GG) \
  if (p.D == DD && G == GG) return launch_plan_t<DD, GG>(p, s);
  KVS_CASE(64, 1) KVS_CASE(64, 2) KVS_CASE(64, 4) KVS_CASE(64, 7) KVS_CASE(64, 8)
  KVS_CASE(128, 1) KVS_CASE(128, 2) KVS_CASE(128, 4) KVS_CASE(128, 7) KVS_CASE(128, 8)
#undef KVS_CASE
  return hipErrorInvalidValue;
}

hipError_t launch_update(const kvskip_update_args& p, hipStream_t s) {
  const int G = p.Hq / p.Hkv;
  switch (G) {
    case 1: return launch_update_t<1>(p, s);
    case 2: return launch_update_t<2>(p, s);
    case 4: return launch_update_t<4>(p, s);
    case 7: return launch_update_t<7>(p, s);
    case 8: return launch_update_t<8>(p, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_block_sums(const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st, int B, int Hkv, int T,
                             int D, float* csum, int NBC, hipStream_t s) {
  const dim3 grid(NBC, Hkv, B);
  const uint16_t* kk = reinterpret_cast<const uint16_t*>(k);
  if (D == 128)
    hipLaunchKernelGGL((block_sums_kernel<128>), grid, dim3(128), 0, s, kk, k_sb, k_sh, k_st, Hkv, T, csum, NBC);
  else if (D == 64)
    hipLaunchKernelGGL((block_sums_kernel<64>), grid, dim3(64), 0, s, kk, k_sb, k_sh, k_st, Hkv, T, csum, NBC);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_token_index(const int32_t* ids, int64_t ids_stride, int B, int T, uint8_t* idx, int NBC,
                              hipStream_t s) {
  const dim3 grid((NBC + 3) / 4, B);
  hipLaunchKernelGGL(token_index_kernel, grid, dim3(256), 0, s, ids, ids_stride, T, idx, NBC);
  return hipGetLastError();
}

}  // namespace kvs
