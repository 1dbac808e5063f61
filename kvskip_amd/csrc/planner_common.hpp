// Device-side refresh planner: helpers shared by the planner kernels and the body of the update
// workgroup, which runs in its own launch, beside the split merge, or beside the next split pass.
#pragma once
#include "attn_common.hpp"

namespace kvs {
namespace {

__device__ __forceinline__ bool always_block(int blk, int nb, int local) { return blk == 0 || blk >= nb - local; }

// Tokens of sequence b: clamp(seq_lens[b], 1, T) in a ragged batch, else T.
__device__ __forceinline__ int seq_T(const int32_t* seq_lens, int b, int T) {
  return seq_lens != nullptr ? min(max(seq_lens[b], 1), T) : T;
}

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

// Whole-wavefront log-sum-exp of per-lane (m, s) pairs: max, then rescaled sums (uniform result).
__device__ __forceinline__ void lse_wave(float& m, float& s) {
  const float M = wave_max(s > 0.f ? m : NEG_INF);
  const float S = wave_sum(s > 0.f ? s * __expf(m - M) : 0.f);
  m = M;
  s = S;
}

constexpr int MAX_NB = 4096;   // planner block capacity: update holds a head's blocks in registers

// Order-preserving key of a float (larger float -> larger key).
__device__ __forceinline__ uint32_t fkey(float y) {
  const uint32_t u = __float_as_uint(y);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Update of (b, KV head h): src/kvskip_attn.py:386-391 (_calib_learn 302-320, _refresh_state
// 182-199, _attended_lse 282-288) on the device, as kernels/kvskip_planner.cu:229-305.
// Wavefront w < NWV takes query heads g = w + NWV j of the group (HPW = ceil(G / NWV) per
// wavefront); lane holds blocks i = lane + 64 r, r < R (nb <= 64 R). Wavefronts >= NWV of a wider
// workgroup only pass the barrier.
template <int G, int R, int NWV>
__device__ __forceinline__ void update_body(const kvskip_update_args& p, int h, int b) {
  constexpr int HPW = (G + NWV - 1) / NWV;
  constexpr int RC = R < 16 ? R : 16;  // register slots whose loads are in flight together
  if (threadIdx.x >= NWV * WAVE) {
    __syncthreads();
    return;
  }
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE;
  const int nbl = (p.T + BLK - 1) / BLK;                       // row length of the statistics
  const int nb = (seq_T(p.seq_lens, b, p.T) + BLK - 1) / BLK;   // the sequence's blocks
  const int64_t bh = static_cast<int64_t>(b) * p.Hkv + h;
  const int64_t hrow0 = static_cast<int64_t>(b) * p.Hq + static_cast<int64_t>(h) * G;  // head g: hrow0 + g
  __shared__ uint64_t sKm[G][R];  // each query head's top-p blocks (lane bits of r)
  __shared__ float sReal[G];
  uint8_t* keep = p.keep + bh * p.NBC;
  const uint8_t* ixp = p.idx != nullptr ? p.idx + static_cast<int64_t>(b) * p.NBC : keep;  // keep: stand-in
  const bool tr = p.trig[bh] != 0;
  const int fl = p.flags != nullptr ? p.flags[h] : 0;
  const bool uni = p.idx != nullptr && ((fl & 4) || (p.aix != nullptr && p.aix[bh] != 0));
  const bool ixh = (fl & 2) != 0;  // token-index head: read index + sink + local (list_stats)
  const float est0 = p.calib != nullptr ? p.est[bh] : 0.f;
  const float cal0 = p.calib != nullptr ? p.calib[bh] : 0.f;

  float x[HPW][R];     // block log-weights blk_max + log blk_sum (-inf where not read / past nb)
  uint64_t kp = 0;     // bit r: block in the stored set before this update
  uint64_t att = 0;    // bit r: block attended this step (stored set + sink + local + index union)
#pragma unroll
  for (int c = 0; c < R; c += RC) {
    float bm[HPW][RC], bs[HPW][RC];
    uint32_t kb[RC], ib[RC];
#pragma unroll
    for (int r = 0; r < RC; ++r) {  // loads of the chunk first, clamped in range
      const int ic = min(lane + WAVE * (c + r), nb - 1);
#pragma unroll
      for (int j = 0; j < HPW; ++j) {
        const int64_t row = hrow0 + min(wave + NWV * j, G - 1);
        bm[j][r] = p.blk_max[row * nbl + ic];
        bs[j][r] = p.blk_sum[row * nbl + ic];
      }
      kb[r] = keep[ic];
      ib[r] = ixp[ic];
    }
#pragma unroll
    for (int r = 0; r < RC; ++r) {
      const int i = lane + WAVE * (c + r);
      const bool in = i < nb;
      const bool al = always_block(i, nb, p.local);
      const bool k = in && kb[r] != 0;
      const bool a = in && (k || al || (uni && ib[r] != 0));
      const bool rd = in && (!p.list_stats || tr || (ixh ? (p.idx != nullptr && ib[r] != 0) || al : a));
#pragma unroll
      for (int j = 0; j < HPW; ++j) x[j][c + r] = rd ? bm[j][r] + __logf(bs[j][r]) : NEG_INF;
      kp |= static_cast<uint64_t>(k) << (c + r);
      att |= static_cast<uint64_t>(a) << (c + r);
    }
  }

  if (tr) {
    // Slots r >= RU hold no block of the sequence (x = -inf): the loops below skip them in
    // groups of 4 (RU uniform).
    const int RU = R <= 4 ? R : __builtin_amdgcn_readfirstlane(min(R, 4 * ((nb + 4 * WAVE - 1) / (4 * WAVE))));
#pragma unroll
    for (int j = 0; j < HPW; ++j) {
      const int g = wave + NWV * j;
      if (g >= G) break;
      const int64_t hrow = hrow0 + g;
      float cn[R <= 16 ? R : 1];  // cs_now of the refresh, in flight during the search
      if constexpr (R <= 16) {
#pragma unroll
        for (int r = 0; r < R; ++r) cn[r] = p.cs_now[hrow * p.NBC + min(lane + WAVE * r, nb - 1)];
      }
      float mx = NEG_INF;
#pragma unroll
      for (int r = 0; r < R; ++r) mx = fmaxf(mx, x[j][r]);
      mx = wave_max(mx);
      float se = 0.f;
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (r < RU) se += __expf(x[j][r] - mx);
      const float lse = mx + __logf(wave_sum(se));
      float w[R];
      uint32_t key[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float y = x[j][r] - lse;
        w[r] = r < RU ? __expf(y) : 0.f;
        key[r] = fkey(y);
      }
      // Largest key theta of y = x - lse whose upper set {key >= theta} holds >= level of the
      // mass: the fewest blocks reaching level (ties at the cut kept); exact, 32 bit steps.
      uint32_t theta = 0;
      for (int bit = 31; bit >= 0; --bit) {
        const uint32_t cand = theta | (1u << bit);
        float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
        for (int r = 0; r < R; r += 2) {
          if (r < RU) {
            acc0 += key[r] >= cand ? w[r] : 0.f;
            if (r + 1 < R) acc1 += key[r + 1] >= cand ? w[r + 1] : 0.f;
          }
        }
        if (wave_sum(acc0 + acc1) >= p.level) theta = cand;
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint64_t m = __ballot(lane + WAVE * r < nb && key[r] >= theta);
        if (lane == 0) sKm[g][r] = m;
      }
      if (p.calib != nullptr) {  // the mass the attended set missed (this head read every block)
        float mi = NEG_INF, si = 0.f, mo = NEG_INF, so = 0.f;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if ((att >> r) & 1)
            lse_push(mi, si, x[j][r]);
          else
            lse_push(mo, so, x[j][r]);
        }
        lse_wave(mi, si);
        lse_wave(mo, so);
        if (lane == 0) sReal[g] = so > 0.f ? 1.f / (1.f + __expf((mi + __logf(si)) - (mo + __logf(so)))) : 0.f;
      }
      // references of the refresh: lse_ref <- x, cs_ref <- cs_now (capacity tail: -inf / 0)
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int i = lane + WAVE * r;
        if (i < p.NBC) {
          float c;
          if constexpr (R <= 16)
            c = cn[r];
          else
            c = p.cs_now[hrow * p.NBC + min(i, nb - 1)];
          p.lse_ref[hrow * p.NBC + i] = x[j][r];
          p.cs_ref[hrow * p.NBC + i] = i < nb ? c : 0.f;
        }
      }
      for (int i = WAVE * R + lane; i < p.NBC; i += WAVE) {
        p.lse_ref[hrow * p.NBC + i] = NEG_INF;
        p.cs_ref[hrow * p.NBC + i] = 0.f;
      }
    }
  }
  __syncthreads();  // every read of the old stored set is done; sKm / sReal complete

  if (tr && p.calib != nullptr && tid == 0) {
    float real = 0.f;
    for (int g = 0; g < G; ++g) real = fmaxf(real, sReal[g]);
    const float resid = p.calib_kind ? real - est0 : clamped_logit(real) - clamped_logit(est0);
    float c = p.calib_kind == 2 ? fmaxf((1.f - p.calib_rate) * cal0, resid)
                                : (1.f - p.calib_rate) * cal0 + p.calib_rate * resid;
    if (!p.calib_free) c = fmaxf(c, 0.f);
    p.calib[bh] = c;
    if (p.aix != nullptr && c > p.aix_thr) p.aix[bh] = 1;
  }
  uint64_t kn = kp;  // bit r: block in the stored set after this update
  if (tr) {
    kn = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      uint64_t u = 0;
#pragma unroll
      for (int g = 0; g < G; ++g) u |= sKm[g][r];
      const int i = lane + WAVE * r;
      const bool k = i < nb && (((u >> lane) & 1) || always_block(i, nb, p.local));
      kn |= static_cast<uint64_t>(k) << r;
      if (wave == r % NWV && i < p.NBC) keep[i] = k ? 1 : 0;
    }
    for (int i = WAVE * R + tid; i < p.NBC; i += NWV * WAVE) keep[i] = 0;
  }
  // Attended log-sum-exp for the next step (every head): the stored set + sink + local.
#pragma unroll
  for (int j = 0; j < HPW; ++j) {
    const int g = wave + NWV * j;
    if (g >= G) break;
    float m2 = NEG_INF, s2 = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int i = lane + WAVE * r;
      if (i < nb && (((kn >> r) & 1) || always_block(i, nb, p.local))) lse_push(m2, s2, x[j][r]);
    }
    lse_wave(m2, s2);
    if (lane == 0) p.lse_att[hrow0 + g] = s2 > 0.f ? m2 + __logf(s2) : NEG_INF;
  }
}

}  // namespace
}  // namespace kvs
