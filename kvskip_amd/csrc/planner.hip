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
// plan:   one workgroup of 16 wavefronts per (b, KV head). Centroid scores with 16 lanes per
//         block row (fp32 key sums, 16 block rows in flight per wavefront); the drift estimate is
//         folded into the same pass (lane 16 r + g keeps head g's running log-sum-exp), so no
//         LDS copy of the scores is needed; every load of a step (key sums, references, set
//         flags, the appended key) is issued before any use; the block list is compacted in
//         ascending order by ballots of the whole workgroup.
// update: one wavefront per query head of the group (G wavefronts), the head's blocks held in
//         registers (64 per register slot). Top-p by an exact bitwise search for the largest
//         score key whose upper set holds >= level of the mass (the fewest blocks reaching
//         level; ties at the threshold are all kept), on weights computed once; wavefront sums
//         stay in DPP rows + readlane; the group's union goes through LDS as ballot masks.
#include "planner_common.hpp"

namespace kvs {
namespace {

constexpr int PW = 16;         // plan workgroup: 16 wavefronts
constexpr int PNT = PW * WAVE;

// Ascending compaction of {i < nb : sF[i] != 0} into out[] by the whole plan workgroup (chunks of
// PNT blocks, wavefront w taking the chunk's w-th 64); returns the count (uniform).
__device__ int compact_wg(const uint8_t* sF, int nb, int* out, int* sCnt) {
  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
  int base = 0;
  for (int c0 = 0; c0 < nb; c0 += PNT) {
    const int i = c0 + tid;
    const bool f = i < nb && sF[i] != 0;
    const uint64_t m = __ballot(f);
    if (lane == 0) sCnt[wave] = __popcll(m);
    __syncthreads();
    int off = base, tot = 0;
#pragma unroll
    for (int w = 0; w < PW; ++w) {
      const int c = sCnt[w];
      off += w < wave ? c : 0;
      tot += c;
    }
    if (f) out[off + __popcll(m & ((uint64_t(1) << lane) - 1))] = i;
    base += tot;
    __syncthreads();
  }
  return base;
}

template <int D, int G>
__global__ void __launch_bounds__(PNT) plan_kernel(const kvskip_plan_args p) {
  constexpr int DL = D / 16;                         // dims per lane: {64 w + 4 c16 + j}
  constexpr int DW = DL / 4;
  constexpr int PU = (D == 128 && G >= 7) ? 2 : 4;  // block-row groups (4 rows each) in flight, 128 VGPRs
  const int h = blockIdx.x, b = blockIdx.y;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE;
  const int Tb = seq_T(p.seq_lens, b, p.T);
  const int nb = (Tb + BLK - 1) / BLK;
  if (p.seq_lens_out != nullptr && h == 0 && tid == 0) p.seq_lens_out[b] = Tb;
  const int64_t bh = static_cast<int64_t>(b) * p.Hkv + h;
  const int64_t row0 = (static_cast<int64_t>(b) * p.Hq + static_cast<int64_t>(h) * G) * p.NBC;  // head g: + g*NBC
  float* csum = p.csum + bh * p.NBC * D;
  const uint8_t* keep = p.keep + bh * p.NBC;
  int* bi = p.block_idx + bh * p.NBC;
  const int fl = p.flags[h];
  __shared__ uint8_t sF[MAX_NB];  // attended set of this step (block flags)
  __shared__ float sM[PW][G], sS[PW][G];
  __shared__ int sCnt[PW];
  __shared__ int sTrig;

  if (fl & 2) {  // token-index head: index blocks + sink + local, never refreshes
    const uint8_t* idx = p.idx != nullptr ? p.idx + static_cast<int64_t>(b) * p.NBC : nullptr;
    for (int i = tid; i < nb; i += PNT)
      sF[i] = ((idx != nullptr && idx[i] != 0) || always_block(i, nb, p.local)) ? 1 : 0;
    __syncthreads();
    const int cnt = compact_wg(sF, nb, bi, sCnt);
    if (tid == 0) {
      p.block_cnt[bh] = cnt;
      p.trig[bh] = 0;
    }
    return;
  }
  const bool uni = p.idx != nullptr && ((fl & 4) || (p.aix != nullptr && p.aix[bh] != 0));
  const uint8_t* ixp = uni ? p.idx + static_cast<int64_t>(b) * p.NBC : keep;  // keep: stand-in
  // decision inputs, in flight during the pass
  const int age0 = p.age[bh];
  const float cal0 = (p.calib != nullptr && p.calib_on) ? p.calib[bh] : 0.f;
  const float la = p.lse_att[static_cast<int64_t>(b) * p.Hq + static_cast<int64_t>(h) * G + min(lane, G - 1)];

  // Lane (rs = lane/16, c16 = lane%16) of a wavefront step: block row 4u + rs of row group u,
  // dims {64 w + 4 c16 + j}; lane c16 = g also keeps query head g's running log-sum-exp of
  // lse_ref + cs - cs_ref over the unattended blocks.
  const int rs = lane >> 4, c16 = lane & 15;
  float qf[G][DL];
  {
    const uint16_t* q = reinterpret_cast<const uint16_t*>(p.q);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const uint16_t* qp = q + b * p.q_sb + (static_cast<int64_t>(h) * G + g) * p.q_sh;
#pragma unroll
      for (int w = 0; w < DW; ++w) {  // 4 adjacent dims per 8-byte load
        const uint2 t = *reinterpret_cast<const uint2*>(qp + 64 * w + 4 * c16);
        qf[g][4 * w] = bf_lo(t.x) * p.scale;
        qf[g][4 * w + 1] = bf_hi(t.x) * p.scale;
        qf[g][4 * w + 2] = bf_lo(t.y) * p.scale;
        qf[g][4 * w + 3] = bf_hi(t.y) * p.scale;
      }
    }
  }
  // The key appended by this step (row T-1, block nb-1) joins its block's sum, in registers.
  const bool add = p.add_token != 0;
  uint2 kx[DW];
  if (add) {
    const uint16_t* kr = key_row(reinterpret_cast<const uint16_t*>(p.k), p.k_sb, p.k_sh, p.k_st, b, h, Tb - 1,
                                 p.block_table, p.bt_stride, p.num_pages);
#pragma unroll
    for (int w = 0; w < DW; ++w)
      kx[w] = kr != nullptr ? *reinterpret_cast<const uint2*>(kr + 64 * w + 4 * c16) : make_uint2(0u, 0u);
  }
  const int gl = min(c16, G - 1);
  float em = NEG_INF, es = 0.f;
  for (int base = 4 * PU * wave; base < nb; base += 4 * PU * PW) {
    float cv[PU][DL];
    float lr[PU], cr[PU];
    bool at[PU];
#pragma unroll
    for (int u = 0; u < PU; ++u) {  // every load of the step first
      const int rc = min(base + 4 * u + rs, nb - 1);
      const float* cp = csum + static_cast<int64_t>(rc) * D;
#pragma unroll
      for (int w = 0; w < DW; ++w) {
        const float4 t = *reinterpret_cast<const float4*>(cp + 64 * w + 4 * c16);
        cv[u][4 * w] = t.x;
        cv[u][4 * w + 1] = t.y;
        cv[u][4 * w + 2] = t.z;
        cv[u][4 * w + 3] = t.w;
      }
      const int64_t r = row0 + static_cast<int64_t>(gl) * p.NBC + rc;
      lr[u] = p.lse_ref[r];
      cr[u] = p.cs_ref[r];
      at[u] = (static_cast<uint32_t>(keep[rc]) | static_cast<uint32_t>(ixp[rc])) != 0;
    }
#pragma unroll
    for (int u = 0; u < PU; ++u) {
      const int blk = base + 4 * u + rs;
      if (add && blk == nb - 1) {
#pragma unroll
        for (int w = 0; w < DW; ++w) {
          cv[u][4 * w] += bf_lo(kx[w].x);
          cv[u][4 * w + 1] += bf_hi(kx[w].x);
          cv[u][4 * w + 2] += bf_lo(kx[w].y);
          cv[u][4 * w + 3] += bf_hi(kx[w].y);
          *reinterpret_cast<float4*>(csum + static_cast<int64_t>(blk) * D + 64 * w + 4 * c16) =
              make_float4(cv[u][4 * w], cv[u][4 * w + 1], cv[u][4 * w + 2], cv[u][4 * w + 3]);
        }
      }
      const float inv_n = 1.f / static_cast<float>(blk == nb - 1 ? Tb - blk * BLK : BLK);
      float mine = 0.f;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float d = 0.f;
#pragma unroll
        for (int j = 0; j < DL; ++j) d = fmaf(qf[g][j], cv[u][j], d);
        d += dpp<DPP_XOR1>(d);
        d += dpp<DPP_XOR2>(d);
        d += dpp<DPP_HALF_MIRROR>(d);
        d += dpp<DPP_MIRROR>(d);
        if (c16 == g) mine = d * inv_n;
      }
      if (blk < nb) {
        const bool a = at[u] || always_block(blk, nb, p.local);
        if (c16 == 0) sF[blk] = a ? 1 : 0;
        if (c16 < G) {
          p.cs_now[row0 + static_cast<int64_t>(c16) * p.NBC + blk] = mine;
          if (!a) lse_push(em, es, lr[u] + mine - cr[u]);
        }
      }
    }
  }
  // merge the 4 block-row slots of each head (lanes c16, 16 + c16, 32 + c16, 48 + c16)
#pragma unroll
  for (int o = 16; o < WAVE; o <<= 1) {
    const float m2 = __shfl_xor(em, o, WAVE), s2 = __shfl_xor(es, o, WAVE);
    lse_merge(em, es, m2, s2);
  }
  if (rs == 0 && c16 < G) {
    sM[wave][c16] = em;
    sS[wave][c16] = es;
  }
  __syncthreads();

  if (wave == 0) {  // decision: miss = max over the group of sigma(est - lse_att)
    float miss = 0.f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float m = lane < PW ? sM[lane][g] : NEG_INF, sv = lane < PW ? sS[lane][g] : 0.f;
      lse_wave(m, sv);
      if (sv > 0.f) {
        const float est = m + __logf(sv);
        miss = fmaxf(miss, 1.f / (1.f + __expf(lane_value(la, g) - est)));
      }
    }
    if (lane == 0) {
      if (p.est != nullptr) p.est[bh] = miss;
      float dec = miss;
      if (p.calib != nullptr && p.calib_on)
        dec = p.calib_kind ? miss + cal0 : 1.f / (1.f + __expf(-(clamped_logit(miss) + cal0)));
      const int a = age0 + 1;
      const bool tr = dec > p.delta || a >= p.max_age || (fl & 1);
      p.age[bh] = tr ? 0 : a;
      p.trig[bh] = tr ? 1 : 0;
      sTrig = tr;
    }
  }
  __syncthreads();

  if (sTrig != 0) {  // refresh: every block
    for (int i = tid; i < nb; i += PNT) bi[i] = i;
    if (tid == 0) p.block_cnt[bh] = nb;
  } else {
    const int cnt = compact_wg(sF, nb, bi, sCnt);
    if (tid == 0) p.block_cnt[bh] = cnt;
  }
}

// The decision of (b, KV head h) from the scores pass's C partials and its block list (one
// wavefront): plan_decide_kernel's body; COH: the partials come from other workgroups of the same
// launch (agent-scope loads).
template <int G, bool COH>
__device__ __forceinline__ void decide_list(const kvskip_plan_args& p, int b, int h, int lane) {
  // The sequence's length, used only after the decision: loaded first through an index the
  // compiler takes for a per-lane one (a vector load, waited for at its use; as a scalar load its
  // wait came before the decision's loads were issued). Without lengths lse_ref stands in (read
  // only here, at least B entries), its value unused.
  int bv = b;
  asm volatile("" : "+v"(bv));
  const int32_t sl = (p.seq_lens != nullptr ? p.seq_lens : reinterpret_cast<const int32_t*>(p.lse_ref))[bv];
  uint32_t mk[DCL];
  const bool tr = decide_head<G, COH>(p, b, h, lane, mk, true, true);
  const int Tb = p.seq_lens != nullptr ? min(max(sl, 1), p.T) : p.T;  // seq_T's rule
  const int nb = (Tb + BLK - 1) / BLK;  // the sequence's blocks
  if (p.seq_lens_out != nullptr && h == 0 && lane == 0) p.seq_lens_out[b] = Tb;
  write_block_list(p, static_cast<int64_t>(b) * p.Hkv + h, nb, tr, mk, lane);
}

// A scores partial written for the decision of the same launch (COH: relaxed agent-scope atomic
// store, which goes past this XCD's L2 to the device's coherence point) or for a later launch.
template <bool COH>
__device__ __forceinline__ void st_part(float* a, float v) {
  if constexpr (COH)
    __hip_atomic_store(reinterpret_cast<uint32_t*>(a), __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else
    *a = v;
}

// The end of a scores workgroup of the one-launch plan (kvskip_plan_args.ticket): once its partial
// stores have completed (s_waitcnt vmcnt(0) in every thread, then the barrier), one agent-scope
// atomic add on the (b, KV head)'s ticket; the workgroup that draws C - 1 (every other partial
// complete before it) decides the head from all C partials, then sets the ticket back to 0 for
// the next call. No workgroup waits for another.
template <int G>
__device__ __forceinline__ void decide_if_last(const kvskip_plan_args& p, int b, int h, int C) {
  __shared__ int sLast;
  const int64_t bh = static_cast<int64_t>(b) * p.Hkv + h;
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this thread's partial stores are complete
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  if (threadIdx.x == 0)
    sLast = __hip_atomic_fetch_add(p.ticket + bh, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == C - 1 ? 1 : 0;
  __syncthreads();
  if (sLast == 0 || threadIdx.x >= WAVE) return;
  decide_list<G, true>(p, b, h, threadIdx.x);
  if (threadIdx.x == 0) __hip_atomic_store(p.ticket + bh, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// FUSED (kvskip_plan_args.ticket set): the one-launch plan, the decision by each head's last
// workgroup (decide_if_last); else the scores pass alone, its partials published by the kernel's end.
template <int D, int G, bool FUSED>
__global__ void __launch_bounds__(WNT) plan_scores_kernel(const kvskip_plan_args p) {
  constexpr int DL = D / 16, DW = DL / 4, SP = part_stride(G);
  // One field of each 64-byte line of the argument block, fetched together up front: read where
  // the code first needs them, the fields' lines came in one after another, a scalar-load wait
  // for each before the pass's loads were issued.
  const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z, C = gridDim.x;
  asm volatile("" ::"s"(p.q), "s"(p.lse_ref), "s"(p.est), "s"(p.part), "s"(p.ids), "s"(C));
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE;
  const int Tb = seq_T(p.seq_lens, b, p.T);
  const int nb = (Tb + BLK - 1) / BLK;
  const int64_t bh = static_cast<int64_t>(b) * p.Hkv + h;
  if (p.seq_lens_out != nullptr && c == 0 && h == 0 && tid == 0) p.seq_lens_out[b] = Tb;  // also when decided in the pass
  if (c * WCB >= nb) {  // a chunk past the sequence's blocks (ragged batch): the empty partial
    float* part = p.part + (bh * C + c) * SP;
    if (tid < G) {
      st_part<FUSED>(part + tid, NEG_INF);
      st_part<FUSED>(part + G + tid, 0.f);
    }
    if (tid == 0) st_part<FUSED>(part + 2 * G, __uint_as_float(0u));
    if constexpr (FUSED) decide_if_last<G>(p, b, h, C);
    return;
  }
  const int64_t row0 = (static_cast<int64_t>(b) * p.Hq + static_cast<int64_t>(h) * G) * p.NBC;
  float* csum = p.csum + bh * p.NBC * D;
  const uint8_t* keep = p.keep + bh * p.NBC;
  // The head's flags and latch are read through indices the compiler takes for per-lane ones: as
  // uniform values they went to scalar registers, a wait for each load before the pass's other loads
  // were issued (the code branching on them was hoisted above those loads).
  int hv = h, bhv = static_cast<int>(bh);
  asm volatile("" : "+v"(hv), "+v"(bhv));
  const int fl = p.flags[hv];
  const bool ixh = (fl & 2) != 0;  // token-index head: index + sink + local, no estimate
  const uint8_t axv = (p.aix != nullptr ? p.aix : p.keep)[bhv];  // p.keep: in-bounds stand-in
  const bool ax = (p.aix != nullptr) & (axv != 0);
  const bool have_ix = p.idx != nullptr || p.ids != nullptr;  // ids: the index is found here
  const bool uni = have_ix & (((fl & 4) != 0) | ax);  // no short circuit: a branch here waited for the loads
  const uint8_t* idx = p.idx != nullptr ? p.idx + static_cast<int64_t>(b) * p.NBC : keep;  // keep: stand-in
  const bool use_idx = have_ix && (ixh || uni);
  __shared__ float sM[WW][G], sS[WW][G];
  __shared__ uint32_t sMask[WW];
  const int base = c * WCB + wave * (4 * WU);  // this wavefront's blocks: base + 4 u + rs

  // Token index (ids given; kvskip_token_index's rule): the wavefront's BPW blocks, LPB lanes per
  // block, lane l checking the TPL tokens TPL (l % LPB) + [0, TPL) of block base + l / LPB (bit i
  // of the result: block base + i); the workgroups of KV head 0 also write them to idx_out for the
  // update. The ids are loaded here and compared after the pass's other loads are issued (the
  // comparison waits for them).
  constexpr int BPW = 4 * WU, LPB = WAVE / BPW, TPL = BLK / LPB;
  const int32_t* ids = p.ids != nullptr ? p.ids + b * p.ids_sb : nullptr;
  const int ix_blk = base + lane / LPB, ix_j0 = ix_blk * BLK + TPL * (lane % LPB);
  int32_t ix_cur = 0, ix_x[TPL + 1];  // the current token; tokens j0 - 1 .. j0 + TPL - 1 (clamped loads)
  if (ids != nullptr) {
    ix_cur = ids[Tb - 1];
#pragma unroll
    for (int e = 0; e <= TPL; ++e) ix_x[e] = ids[min(max(ix_j0 - 1 + e, 0), Tb - 1)];
  }

  // Every load is issued without waiting for the flags (an index head's extra loads are unused).
  const int rs = lane >> 4, c16 = lane & 15, gl = min(c16, G - 1);
  float qf[G][DL];
  uint2 kx[DW];
  bool have_kr = true;
  {
    const uint16_t* q = reinterpret_cast<const uint16_t*>(p.q);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const uint16_t* qp = q + b * p.q_sb + (static_cast<int64_t>(h) * G + g) * p.q_sh;
#pragma unroll
      for (int w = 0; w < DW; ++w) {  // 4 adjacent dims per 8-byte load
        const uint2 t = *reinterpret_cast<const uint2*>(qp + 64 * w + 4 * c16);
        qf[g][4 * w] = bf_lo(t.x) * p.scale;
        qf[g][4 * w + 1] = bf_hi(t.x) * p.scale;
        qf[g][4 * w + 2] = bf_lo(t.y) * p.scale;
        qf[g][4 * w + 3] = bf_hi(t.y) * p.scale;
      }
    }
    // the appended key row (none on an invalid page: read from the pool's first row, added as zeros),
    // loaded unconditionally so that no wait for it precedes the loads below
    const uint16_t* kr = key_row(reinterpret_cast<const uint16_t*>(p.k), p.k_sb, p.k_sh, p.k_st, b, h, Tb - 1,
                                 p.block_table, p.bt_stride, p.num_pages);
    have_kr = kr != nullptr;
    const uint16_t* krs = have_kr ? kr : reinterpret_cast<const uint16_t*>(p.k);
#pragma unroll
    for (int w = 0; w < DW; ++w) kx[w] = *reinterpret_cast<const uint2*>(krs + 64 * w + 4 * c16);
  }
  const bool add = p.add_token != 0 && !ixh;

  float cv[WU][DL], lr[WU], cr[WU];
  uint32_t kb[WU], ib[WU];
#pragma unroll
  for (int u = 0; u < WU; ++u) {  // every load of the pass first
    const int rc = min(base + 4 * u + rs, nb - 1);
    {
      const float* cp = csum + static_cast<int64_t>(rc) * D;
#pragma unroll
      for (int w = 0; w < DW; ++w) {
        const float4 t = *reinterpret_cast<const float4*>(cp + 64 * w + 4 * c16);
        cv[u][4 * w] = t.x;
        cv[u][4 * w + 1] = t.y;
        cv[u][4 * w + 2] = t.z;
        cv[u][4 * w + 3] = t.w;
      }
      const int64_t r = row0 + static_cast<int64_t>(gl) * p.NBC + rc;
      lr[u] = p.lse_ref[r];
      cr[u] = p.cs_ref[r];
    }
    kb[u] = keep[rc];
    ib[u] = ids != nullptr ? 0u : idx[rc];
  }
  if (ids != nullptr) {
    bool hit = false;
#pragma unroll
    for (int e = 1; e <= TPL; ++e) {
      const int j = ix_j0 + e - 1;
      hit |= (j < Tb - 1 && ix_x[e] == ix_cur) || (j < Tb && j >= 1 && ix_x[e - 1] == ix_cur);
    }
    const uint64_t bal = __ballot(hit);
    constexpr uint64_t LM = LPB == WAVE ? ~uint64_t(0) : (uint64_t(1) << LPB) - 1;
    uint32_t ixw = 0;
#pragma unroll
    for (int i = 0; i < BPW; ++i) ixw |= ((bal >> (LPB * i)) & LM) != 0 ? 1u << i : 0u;
    if (h == 0 && lane % LPB == 0 && ix_blk < nb)
      p.idx_out[static_cast<int64_t>(b) * p.NBC + ix_blk] = (ixw >> (lane / LPB)) & 1;
#pragma unroll
    for (int u = 0; u < WU; ++u) ib[u] = (ixw >> (4 * u + rs)) & 1;
  }
  float em = NEG_INF, es = 0.f;
  uint32_t wmask = 0;  // attended blocks of this wavefront: bit 4 u + rs
#pragma unroll
  for (int u = 0; u < WU; ++u) {
    const int blk = base + 4 * u + rs;
    const bool in = blk < nb, al = always_block(blk, nb, p.local);
    const bool a = in && (ixh ? (use_idx && ib[u] != 0) || al : kb[u] != 0 || al || (uni && ib[u] != 0));
    const uint64_t bal = __ballot(c16 == 0 && a);
    wmask |= static_cast<uint32_t>(((bal >> 0) & 1) | (((bal >> 16) & 1) << 1) | (((bal >> 32) & 1) << 2) |
                                   (((bal >> 48) & 1) << 3)) << (4 * u);
    if (ixh) continue;
    if (add && blk == nb - 1) {
#pragma unroll
      for (int w = 0; w < DW; ++w) {
        const uint2 kv = have_kr ? kx[w] : make_uint2(0u, 0u);
        cv[u][4 * w] += bf_lo(kv.x);
        cv[u][4 * w + 1] += bf_hi(kv.x);
        cv[u][4 * w + 2] += bf_lo(kv.y);
        cv[u][4 * w + 3] += bf_hi(kv.y);
        *reinterpret_cast<float4*>(csum + static_cast<int64_t>(blk) * D + 64 * w + 4 * c16) =
            make_float4(cv[u][4 * w], cv[u][4 * w + 1], cv[u][4 * w + 2], cv[u][4 * w + 3]);
      }
    }
    const float inv_n = 1.f / static_cast<float>(blk == nb - 1 ? Tb - blk * BLK : BLK);
    float mine = 0.f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float d = 0.f;
#pragma unroll
      for (int j = 0; j < DL; ++j) d = fmaf(qf[g][j], cv[u][j], d);
      d += dpp<DPP_XOR1>(d);
      d += dpp<DPP_XOR2>(d);
      d += dpp<DPP_HALF_MIRROR>(d);
      d += dpp<DPP_MIRROR>(d);
      if (c16 == g) mine = d * inv_n;
    }
    if (in && c16 < G) {
      p.cs_now[row0 + static_cast<int64_t>(c16) * p.NBC + blk] = mine;
      if (!a) lse_push(em, es, lr[u] + mine - cr[u]);
    }
  }
#pragma unroll
  for (int o = 16; o < WAVE; o <<= 1) {
    const float m2 = __shfl_xor(em, o, WAVE), s2 = __shfl_xor(es, o, WAVE);
    lse_merge(em, es, m2, s2);
  }
  if (rs == 0 && c16 < G) {
    sM[wave][c16] = em;
    sS[wave][c16] = es;
  }
  if (lane == 0) sMask[wave] = wmask;
  __syncthreads();
  float* part = p.part + (bh * C + c) * SP;
  if (wave == 0 && lane < G) {
    float m = NEG_INF, sv = 0.f;
#pragma unroll
    for (int w = 0; w < WW; ++w) lse_merge(m, sv, sM[w][lane], sS[w][lane]);
    st_part<FUSED>(part + lane, m);
    st_part<FUSED>(part + G + lane, sv);
  }
  if (tid == 0) {
    uint32_t mk = 0;
#pragma unroll
    for (int w = 0; w < WW; ++w) mk |= sMask[w] << (BPW * w);
    st_part<FUSED>(part + 2 * G, __uint_as_float(mk));
  }
  if constexpr (FUSED) decide_if_last<G>(p, b, h, C);
}

// One wavefront per (b, KV head): the decision from the C = ceil(nb / 32) partials (decide_head,
// the arithmetic the planned pass's prologue repeats) and the list compacted from the chunk masks.
template <int G>
__global__ void __launch_bounds__(WAVE) plan_decide_kernel(const kvskip_plan_args p) {
  decide_list<G, false>(p, blockIdx.y, blockIdx.x, threadIdx.x);
}

template <int G, int R>
__global__ void __launch_bounds__(G * WAVE) update_kernel(const kvskip_update_args p) {
  update_body<G, R, G>(p, blockIdx.x, blockIdx.y);
}

// One launch for the split merge of the attention pass and the update of the planner: workgroups
// [0, B Hkv) update (first, so their longer latency chain starts at once), the next B Hq D/32
// merge (both read only what the split pass wrote).
constexpr int fused_threads(int G) { return G * WAVE > 256 ? G * WAVE : 256; }

template <int D, int G, int R>
__global__ void __launch_bounds__(fused_threads(G)) merge_update_kernel(const AttnP a, const kvskip_update_args u) {
  const int n_update = u.B * u.Hkv;
  const int i = blockIdx.x;
  if (i < n_update) {
    update_body<G, R, G>(u, i % u.Hkv, i / u.Hkv);
  } else {
    const int j = i - n_update;
    merge_body_rt<D>(a, j / (D / 32), j % (D / 32));
  }
}

// csum[b, h, blk, d] = sum over the block's rows t < T_b of k[b, h, t, d]; zero for blk >= nb_b.
// 256 threads: thread (row group rg, 4-dim column c) adds its 64 / RG rows, all loads in flight,
// then the RG partial rows are added in LDS (in row-group order).
template <int D>
__global__ void __launch_bounds__(256) block_sums_kernel(const uint16_t* k, int64_t k_sb, int64_t k_sh,
                                                         int64_t k_st, int Hkv, int T, float* csum, int NBC,
                                                         const int32_t* seq_lens, const int32_t* tbl, int64_t bt,
                                                         int npages) {
  constexpr int DL = D / 4, RG = 256 / DL, RPT = BLK / RG;
  const int blk = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, rg = tid / DL, c = tid % DL;
  const int Tb = seq_T(seq_lens, b, T);
  // the block's first row (its page's, with a block table; an invalid page sums to zero)
  const uint16_t* kb = blk * BLK < Tb ? key_row(k, k_sb, k_sh, k_st, b, h, blk * BLK, tbl, bt, npages) : nullptr;
  __shared__ float part[RG][D];
  uint2 x[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int r = rg + RG * i;
    x[i] = (kb != nullptr && blk * BLK + r < Tb) ? *reinterpret_cast<const uint2*>(kb + 4 * c + static_cast<int64_t>(r) * k_st)
                                               : make_uint2(0u, 0u);
  }
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    a0 += bf_lo(x[i].x);
    a1 += bf_hi(x[i].x);
    a2 += bf_lo(x[i].y);
    a3 += bf_hi(x[i].y);
  }
  part[rg][4 * c] = a0;
  part[rg][4 * c + 1] = a1;
  part[rg][4 * c + 2] = a2;
  part[rg][4 * c + 3] = a3;
  __syncthreads();
  if (tid < D) {
    float a = 0.f;
#pragma unroll
    for (int r = 0; r < RG; ++r) a += part[r][tid];
    csum[((static_cast<int64_t>(b) * Hkv + h) * NBC + blk) * D + tid] = a;
  }
}

// idx[b, blk] = any position j < T of the block with ids[j] == cur (j < T-1) or ids[j-1] == cur
// (j-1 < T-1), cur = ids[T-1]. One wavefront per block, lane = token.
__global__ void __launch_bounds__(256) token_index_kernel(const int32_t* ids, int64_t stride, int Tcap, uint8_t* idx,
                                                          int NBC, const int32_t* seq_lens) {
  const int b = blockIdx.y;
  const int blk = blockIdx.x * 4 + threadIdx.x / WAVE;
  const int lane = threadIdx.x % WAVE;
  if (blk >= NBC) return;
  const int T = seq_T(seq_lens, b, Tcap);
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
  if (p.part != nullptr && p.ticket != nullptr) {
    const int nb = (p.T + BLK - 1) / BLK;
    hipLaunchKernelGGL((plan_scores_kernel<D, G, true>), dim3((nb + WCB - 1) / WCB, p.Hkv, p.B), dim3(WNT), 0, s, p);
  } else if (p.part != nullptr) {
    const int nb = (p.T + BLK - 1) / BLK;
    hipLaunchKernelGGL((plan_scores_kernel<D, G, false>), dim3((nb + WCB - 1) / WCB, p.Hkv, p.B), dim3(WNT), 0, s, p);
    hipLaunchKernelGGL((plan_decide_kernel<G>), dim3(p.Hkv, p.B), dim3(WAVE), 0, s, p);
  } else {
    hipLaunchKernelGGL((plan_kernel<D, G>), dim3(p.Hkv, p.B), dim3(PNT), 0, s, p);
  }
  return hipGetLastError();
}

template <int G>
hipError_t launch_update_t(const kvskip_update_args& p, hipStream_t s) {
  const int nb = (p.T + BLK - 1) / BLK;
  const dim3 grid(p.Hkv, p.B), blk(G * WAVE);
  if (nb <= 2 * WAVE) hipLaunchKernelGGL((update_kernel<G, 2>), grid, blk, 0, s, p);
  else if (nb <= 4 * WAVE) hipLaunchKernelGGL((update_kernel<G, 4>), grid, blk, 0, s, p);
  else if (nb <= 8 * WAVE) hipLaunchKernelGGL((update_kernel<G, 8>), grid, blk, 0, s, p);
  else if (nb <= 16 * WAVE) hipLaunchKernelGGL((update_kernel<G, 16>), grid, blk, 0, s, p);
  else if (nb <= 24 * WAVE) hipLaunchKernelGGL((update_kernel<G, 24>), grid, blk, 0, s, p);
  else if (nb <= 32 * WAVE) hipLaunchKernelGGL((update_kernel<G, 32>), grid, blk, 0, s, p);
  else if (nb <= 64 * WAVE) hipLaunchKernelGGL((update_kernel<G, 64>), grid, blk, 0, s, p);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

template <int D, int G>
hipError_t launch_merge_update_t(const AttnP& a, const kvskip_update_args& p, hipStream_t s) {
  const int nb = (p.T + BLK - 1) / BLK;
  const dim3 grid(a.B * a.Hq * (D / 32) + p.B * p.Hkv), blk(fused_threads(G));
  if (nb <= 2 * WAVE) hipLaunchKernelGGL((merge_update_kernel<D, G, 2>), grid, blk, 0, s, a, p);
  else if (nb <= 4 * WAVE) hipLaunchKernelGGL((merge_update_kernel<D, G, 4>), grid, blk, 0, s, a, p);
  else if (nb <= 8 * WAVE) hipLaunchKernelGGL((merge_update_kernel<D, G, 8>), grid, blk, 0, s, a, p);
  else if (nb <= 16 * WAVE) hipLaunchKernelGGL((merge_update_kernel<D, G, 16>), grid, blk, 0, s, a, p);
  else {  // > 1024 blocks: two launches (at 1025 blocks, B 32, the fused form took 77 us against
          // 9 + 30 us for the merge and the update apart: its updates' load chains under the merge's
          // traffic)
    const hipError_t e = launch_combine(a, D, false, s);
    if (e != hipSuccess) return e;
    return launch_update_t<G>(p, s);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_merge_update(const AttnP& a, const kvskip_update_args& p, int D, hipStream_t s) {
  const int G = p.Hq / p.Hkv;
#define KVS_CASE(DD, GG) \
  if (D == DD && G == GG) return launch_merge_update_t<DD, GG>(a, p, s);
  KVS_CASE(64, 1) KVS_CASE(64, 2) KVS_CASE(64, 4) KVS_CASE(64, 7) KVS_CASE(64, 8)
  KVS_CASE(128, 1) KVS_CASE(128, 2) KVS_CASE(128, 4) KVS_CASE(128, 7) KVS_CASE(128, 8)
#undef KVS_CASE
  return hipErrorInvalidValue;
}

// Blocks per head the planner kernels hold (plan: LDS flags; update: registers), any G.
int planner_max_blocks(int) { return MAX_NB; }

int64_t plan_part_floats(int B, int Hq, int Hkv, int NBC) {
  const int G = Hq / Hkv;
  return static_cast<int64_t>(B) * Hkv * ((NBC + WCB - 1) / WCB) * part_stride(G);
}

hipError_t launch_plan(const kvskip_plan_args& p, hipStream_t s) {
  const int G = p.Hq / p.Hkv;
#define KVS_CASE(DD, GG) \
  if (p.D == DD && G == GG) return launch_plan_t<DD, GG>(p, s);
  KVS_CASE(64, 1) KVS_CASE(64, 2) KVS_CASE(64, 4) KVS_CASE(64, 7) KVS_CASE(64, 8)
  KVS_CASE(128, 1) KVS_CASE(128, 2) KVS_CASE(128, 4) KVS_CASE(128, 7) KVS_CASE(128, 8)
#undef KVS_CASE
  return hipErrorInvalidValue;
}

hipError_t launch_plan_scores(const kvskip_plan_args& p, hipStream_t s) {
  const int G = p.Hq / p.Hkv;
  const int nb = (p.T + BLK - 1) / BLK;
#define KVS_CASE(DD, GG)                                                                                     \
  if (p.D == DD && G == GG) {                                                                                \
    hipLaunchKernelGGL((plan_scores_kernel<DD, GG, false>), dim3((nb + WCB - 1) / WCB, p.Hkv, p.B), dim3(WNT), 0, s, p); \
    return hipGetLastError();                                                                                \
  }
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
                             int D, float* csum, int NBC, const int32_t* seq_lens, const int32_t* tbl, int64_t bt,
                             int npages, hipStream_t s) {
  const dim3 grid(NBC, Hkv, B);
  const uint16_t* kk = reinterpret_cast<const uint16_t*>(k);
  if (D == 128)
    hipLaunchKernelGGL((block_sums_kernel<128>), grid, dim3(256), 0, s, kk, k_sb, k_sh, k_st, Hkv, T, csum, NBC,
                       seq_lens, tbl, bt, npages);
  else if (D == 64)
    hipLaunchKernelGGL((block_sums_kernel<64>), grid, dim3(256), 0, s, kk, k_sb, k_sh, k_st, Hkv, T, csum, NBC,
                       seq_lens, tbl, bt, npages);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_token_index(const int32_t* ids, int64_t ids_stride, int B, int T, uint8_t* idx, int NBC, const int32_t* seq_lens,
                              hipStream_t s) {
  const dim3 grid((NBC + 3) / 4, B);
  hipLaunchKernelGGL(token_index_kernel, grid, dim3(256), 0, s, ids, ids_stride, T, idx, NBC, seq_lens);
  return hipGetLastError();
}

}  // namespace kvs
