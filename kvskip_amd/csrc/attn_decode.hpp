// Split-K decode attention, the body of one workgroup: dense or over block lists, with optional
// per-block statistics, stats-only (K only) and fp16 P; both QK engines (MFMA, VALU dot2). Used
// by the decode kernels and by the planner's split pass that carries an update.
#pragma once
#include "planner_common.hpp"

namespace kvs {
namespace {

// Blocks strictly between list entries prev and cur, clipped to [0, nb): [a, a + len), none if
// len <= 0. Both entries are clamped first, so no entry value (a caller's list is not validated
// on the device) can overflow the arithmetic or reach outside the head's statistics.
__host__ __device__ __forceinline__ void gap_range(int prev, int cur, int nb, int& a, int& len) {
  prev = prev < -1 ? -1 : (prev > nb - 1 ? nb - 1 : prev);
  cur = cur < 0 ? 0 : (cur > nb ? nb : cur);
  a = prev + 1;
  len = cur - a;
}

// Masked statistics of the blocks the list skips: (-inf, 0), so the outputs need no fill. The
// split holding list positions [i0, i0 + n) writes the gap before each of its entries (from the
// previous entry, or from block 0) and, if it holds the list's last entry, the tail up to nb;
// an empty list is written by split 0. Every unlisted block falls to exactly one split.
// Wavefront w takes positions i0 + w + NWAVE j; its lane j < 64 holds that entry and the one
// before it (cur0, prev0: loaded at the start of the pass, written after it, so these stores
// overlap the partial results' instead of delaying them).
template <int G, class List>
__device__ void write_gap_stats(const AttnP& p, const List& list, int n_items, int i0, int n, int split,
                                int64_t hq0, int wave, int lane, int prev0, int cur0) {
  // blocks a .. a + len - 1, thread t of a team of `stride`: blocks over the team, the G heads in an
  // unrolled loop (no division by the run-time length)
  auto put_range = [&](int a, int len, int t, int stride) {
    for (int x = t; x < len; x += stride) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        p.blk_max[(hq0 + g) * p.nb + a + x] = NEG_INF;
        p.blk_sum[(hq0 + g) * p.nb + a + x] = 0.f;
      }
    }
  };
  const int tid = wave * WAVE + lane;
  if (n_items == 0) {
    if (split == 0) put_range(0, p.nb, tid, NT);
    return;
  }
  for (int j = 0; wave + NWAVE * j < n; ++j) {  // uniform over the wavefront
    int prev, cur;
    if (j < WAVE) {
      prev = __builtin_amdgcn_readlane(prev0, j);
      cur = __builtin_amdgcn_readlane(cur0, j);
    } else {
      const int k = i0 + wave + NWAVE * j;
      cur = __builtin_amdgcn_readfirstlane(list(k));
      prev = __builtin_amdgcn_readfirstlane(list(k - 1));
    }
    int a, len;
    gap_range(prev, cur, p.nb, a, len);
    put_range(a, len, lane, WAVE);
  }
  if (n > 0 && i0 + n == n_items) {
    const int a = min(max(list(n_items - 1), -1), p.nb - 1) + 1, len = p.nb - a;
    put_range(a, len, tid, NT);
  }
}

// A planned pass over all B * Hkv (<= BAL_MAX_LISTS) lists together (kvskip_plan_args.pass_budget
// > 0): wavefront w decides lists w + NWAVE j together (decide_heads: one load round trip;
// workgroup 0 stores trig and est), the
// lists are cut into chunks of one length C over all of them (pass_budget workgroups' worth, at
// most p.num_splits chunks per list, at least one) numbered list by list, and this workgroup takes
// chunk number bid: its list (b, h), chunk (the partial slot `split`), positions
// [i0, i0 + n) of n_items, refresh flag and, for a stored-set list, its slice of the positions in
// sPl (positions i0 - 1 .. i0 + n - 1). The workgroup of a list's chunk 0 empties the list's unused
// partial slots; on the one of its last chunk, `writer` is set on the wavefront that decided the
// list, whose masks go to omk: it writes the list and its count after its blocks. Returns false for
// a workgroup past the last chunk (nothing to do). Uniform results.
constexpr int BAL_MAX_LISTS = 16;

template <int G, int NH>
__device__ bool planned_balanced_nh(const AttnP& p, const kvskip_plan_args& pa, int bid, int wave, int lane, int nbb,
                                    int* sPl, uint32_t* sMk, int* sPre, int& split, int& h, int& b, int& n_items,
                                    int& i0, int& n, bool& dense, bool& writer, uint32_t (&omk)[DCL]) {
  __shared__ int sCnt[BAL_MAX_LISTS];
  __shared__ int sTr[BAL_MAX_LISTS];
  const int P = p.B * p.Hkv;
  int lists[NH];  // this wavefront's lists wave + NWAVE k (clamped: a repeat is decided, not stored)
#pragma unroll
  for (int k = 0; k < NH; ++k) lists[k] = min(wave + NWAVE * k, P - 1);
  uint32_t mk[NH][DCL];
  bool tr[NH];
  decide_heads<G, NH>(pa, lists, lane, mk, tr, bid == 0 && pa.decide_mode != DECIDE_LISTS, false);
  apply_decide_mode<NH>(pa.decide_mode, mk, tr, lane, nbb);
#pragma unroll
  for (int k = 0; k < NH; ++k) {
    int c = 0;
#pragma unroll
    for (int d = 0; d < DCL; ++d) c += __popc(mk[k][d]);
    c = static_cast<int>(wave_sum(static_cast<float>(c)));  // exact: counts <= MAX_NB
    if (lane == 0 && wave + NWAVE * k < P) {
      sCnt[wave + NWAVE * k] = tr[k] ? nbb : c;
      sTr[wave + NWAVE * k] = tr[k] ? 1 : 0;
    }
  }
  __syncthreads();
  // the partition, lane q holding list q (every wavefront computes the same)
  const int cq = lane < P ? sCnt[lane] : 0;
  const int total = static_cast<int>(wave_sum(static_cast<float>(cq)));  // exact: <= 16 * MAX_NB
  const int most = static_cast<int>(wave_max(static_cast<float>(cq)));
  const int slots = pa.slot_count > 0 ? pa.slot_count : p.num_splits, budget = pa.pass_budget;
  const int C = max(1, max((total + budget - 1) / budget, (most + slots - 1) / slots));
  const int ch = lane < P ? max(1, (cq + C - 1) / C) : 0;
  const int incl = wave_incl_scan(ch);
  const int it = bid;  // consecutive chunks on different XCDs: a grid's unused tail idles no XCD
  const uint64_t hit = __ballot(lane < P && it >= incl - ch && it < incl);
  if (hit == 0) return false;
  const int q_sel = __builtin_ctzll(hit);
  const int ch_sel = __builtin_amdgcn_readlane(ch, q_sel);
  split = it - (__builtin_amdgcn_readlane(incl, q_sel) - ch_sel);
  b = q_sel / p.Hkv;
  h = q_sel % p.Hkv;
  n_items = __builtin_amdgcn_readlane(cq, q_sel);
  dense = sTr[q_sel] != 0;
  i0 = min(n_items, split * C);
  n = min(n_items, i0 + C) - i0;
  writer = false;  // the list's last chunk writes the list at its end (it has the fewest items)
#pragma unroll
  for (int k = 0; k < NH; ++k) {
    if (wave + NWAVE * k == q_sel) {  // the wavefront that decided this list holds its masks
      if (!dense) {
        int pre[DCL];
        mask_prefix(mk[k], lane, plan_chunks(pa.T), pre);
#pragma unroll
        for (int d = 0; d < DCL; ++d) {
          sMk[lane + WAVE * d] = mk[k][d];
          sPre[lane + WAVE * d] = pre[d];
        }
      }
      writer = split == ch_sel - 1;
#pragma unroll
      for (int d = 0; d < DCL; ++d) omk[d] = mk[k][d];
    }
  }
  if (split == 0) {  // the slots [ch_sel, slots) of the list's query heads: empty partials
    const int64_t hq0 = static_cast<int64_t>(b) * p.Hq + static_cast<int64_t>(h) * G;
    for (int t = threadIdx.x; t < G * (slots - ch_sel); t += NT) {
      float* ml = p.part_ml + ((hq0 + t % G) * p.num_splits + pa.slot_base + ch_sel + t / G) * 2;
      ml[0] = NEG_INF;
      ml[1] = 0.f;
    }
  }
  if (!dense) {  // this workgroup's slice, positions i0 - 1 .. i0 + n - 1, by every thread
    __syncthreads();  // the masks and prefixes in LDS
    slice_from_masks(sMk, sPre, plan_chunks(pa.T), i0, i0 + n, sPl, threadIdx.x, NT);
    if (threadIdx.x == 0 && i0 == 0) sPl[0] = -1;
    __syncthreads();
  }
  return true;
}

template <int G>
__device__ bool planned_balanced(const AttnP& p, const kvskip_plan_args& pa, int bid, int wave, int lane, int nbb,
                                 int* sPl, uint32_t* sMk, int* sPre, int& split, int& h, int& b, int& n_items,
                                 int& i0, int& n, bool& dense, bool& writer, uint32_t (&omk)[DCL]) {
  const int P = p.B * p.Hkv;
  if (P <= NWAVE)
    return planned_balanced_nh<G, 1>(p, pa, bid, wave, lane, nbb, sPl, sMk, sPre, split, h, b, n_items, i0, n, dense,
                                     writer, omk);
  if (P <= 2 * NWAVE)
    return planned_balanced_nh<G, 2>(p, pa, bid, wave, lane, nbb, sPl, sMk, sPre, split, h, b, n_items, i0, n, dense,
                                     writer, omk);
  return planned_balanced_nh<G, BAL_MAX_LISTS / NWAVE>(p, pa, bid, wave, lane, nbb, sPl, sMk, sPre, split, h, b,
                                                        n_items, i0, n, dense, writer, omk);
}

// A planned pass over a ragged batch (seq_lens, B <= BAL_MAX_LISTS): workgroup `it` of KV head h
// decides the head's B lists (b, h) in its prologue (wavefront w: b = w + NWAVE j; the head's
// workgroup 0 stores trig and est) and takes chunk `it` of the ragged partition over their lengths
// (a refreshing list: the sequence's blocks; each list cut into ceil(n / C) chunks of near-equal
// length, C ragged_chunk_len's, numbered sequence by sequence, as ragged_lookup and decode_body do
// over the block counts this pass writes, so that the ragged merge finds the same chunks). Outputs as planned_balanced_nh's, plus the sequence's length
// Tb and blocks nbb; the head's workgroup 0 also writes the statistics and the zero count of a list
// with nothing to read. Returns false for a workgroup past the head's chunks. Uniform results.
template <int G, int NH>
__device__ bool planned_ragged_nh(const AttnP& p, const kvskip_plan_args& pa, int h, int it, int wave, int lane,
                                  int* sPl, uint32_t* sMk, int* sPre, int& split, int& b, int& n_items, int& i0,
                                  int& n, bool& dense, bool& writer, uint32_t (&omk)[DCL], int& Tb, int& nbb) {
  __shared__ int sCnt[BAL_MAX_LISTS];
  __shared__ int sTr[BAL_MAX_LISTS];
  const int B = p.B;
  int lists[NH], nbl[NH];  // this wavefront's lists (clamped: a repeat is decided, not stored)
#pragma unroll
  for (int k = 0; k < NH; ++k) {
    const int bb = min(wave + NWAVE * k, B - 1);
    lists[k] = bb * p.Hkv + h;
    nbl[k] = (seq_len(p, bb) + BLK - 1) / BLK;
  }
  uint32_t mk[NH][DCL];
  bool tr[NH];
  decide_heads<G, NH>(pa, lists, lane, mk, tr, it == 0 && pa.decide_mode != DECIDE_LISTS, false);
  apply_decide_mode<NH>(pa.decide_mode, mk, tr, lane, 0);  // PLAN or LISTS (POST is not ragged)
#pragma unroll
  for (int k = 0; k < NH; ++k) {
    int c = 0;
#pragma unroll
    for (int d = 0; d < DCL; ++d) c += __popc(mk[k][d]);
    c = wave_sum_int(c);
    if (lane == 0 && wave + NWAVE * k < B) {
      sCnt[wave + NWAVE * k] = tr[k] ? nbl[k] : c;
      sTr[wave + NWAVE * k] = tr[k] ? 1 : 0;
    }
  }
  __syncthreads();
  // the partition, lane q holding list q (every wavefront computes the same; ragged_chunk_len's
  // length over these counts, which the list writers leave in block_cnt for the merge)
  const int cq = lane < B ? sCnt[lane] : 0;
  const int tot = wave_sum_int(cq);
  const int most = static_cast<int>(wave_max(static_cast<float>(cq)));  // exact: counts <= 2^24
  const int S = p.num_splits;
  int nvq[NRB] = {};
  nvq[0] = cq;
  const int C = fit_chunk_len(p, nvq, B, max(max(1, (most + S - 1) / S), (tot + S + B - 1) / (S + B)),
                              __builtin_amdgcn_readfirstlane(max(1, (tot + S - 1) / S)), S + B);
  const int ch = (cq + C - 1) / C;  // none for an empty list
  const int incl = wave_incl_scan(ch);
  if (it == 0) {  // the head's lists with nothing to read: statistics (-inf, 0) and count 0
    uint64_t empty = __ballot(lane < B && cq == 0);
    while (empty != 0) {
      const int be = __builtin_ctzll(empty);
      empty &= empty - 1;
      if (wave == 0 && lane == 0) pa.block_cnt[static_cast<int64_t>(be) * p.Hkv + h] = 0;
      const int64_t q0 = static_cast<int64_t>(be) * p.Hq + static_cast<int64_t>(h) * G;
      for (int t = threadIdx.x; t < G * p.nb; t += NT) {
        p.blk_max[(q0 + t / p.nb) * p.nb + t % p.nb] = NEG_INF;
        p.blk_sum[(q0 + t / p.nb) * p.nb + t % p.nb] = 0.f;
      }
    }
  }
  const uint64_t hit = __ballot(lane < B && ch > 0 && it >= incl - ch && it < incl);
  if (hit == 0) return false;
  const int q_sel = __builtin_ctzll(hit);
  const int ch_sel = __builtin_amdgcn_readlane(ch, q_sel);
  split = it - (__builtin_amdgcn_readlane(incl, q_sel) - ch_sel);
  b = q_sel;
  n_items = __builtin_amdgcn_readlane(cq, q_sel);
  dense = sTr[q_sel] != 0;
  i0 = split * n_items / ch_sel;  // the list's ch_sel chunks of near-equal length, as decode_body's
  n = (split + 1) * n_items / ch_sel - i0;
  Tb = seq_len(p, b);
  nbb = (Tb + BLK - 1) / BLK;
  writer = false;  // the list's last chunk writes the list at its end
#pragma unroll
  for (int k = 0; k < NH; ++k) {
    if (wave + NWAVE * k == q_sel) {  // the wavefront that decided this list holds its masks
      if (!dense) {
        int pre[DCL];
        mask_prefix(mk[k], lane, plan_chunks(pa.T), pre);
#pragma unroll
        for (int d = 0; d < DCL; ++d) {
          sMk[lane + WAVE * d] = mk[k][d];
          sPre[lane + WAVE * d] = pre[d];
        }
      }
      writer = split == ch_sel - 1;
#pragma unroll
      for (int d = 0; d < DCL; ++d) omk[d] = mk[k][d];
    }
  }
  if (!dense) {  // this workgroup's slice, positions i0 - 1 .. i0 + n - 1, by every thread
    __syncthreads();  // the masks and prefixes in LDS
    slice_from_masks(sMk, sPre, plan_chunks(pa.T), i0, i0 + n, sPl, threadIdx.x, NT);
    if (threadIdx.x == 0 && i0 == 0) sPl[0] = -1;
    __syncthreads();
  }
  return true;
}

template <int G>
__device__ bool planned_ragged(const AttnP& p, const kvskip_plan_args& pa, int h, int it, int wave, int lane,
                               int* sPl, uint32_t* sMk, int* sPre, int& split, int& b, int& n_items, int& i0, int& n,
                               bool& dense, bool& writer, uint32_t (&omk)[DCL], int& Tb, int& nbb) {
  if (p.B <= NWAVE)
    return planned_ragged_nh<G, 1>(p, pa, h, it, wave, lane, sPl, sMk, sPre, split, b, n_items, i0, n, dense, writer,
                                   omk, Tb, nbb);
  if (p.B <= 2 * NWAVE)
    return planned_ragged_nh<G, 2>(p, pa, h, it, wave, lane, sPl, sMk, sPre, split, b, n_items, i0, n, dense, writer,
                                   omk, Tb, nbb);
  return planned_ragged_nh<G, BAL_MAX_LISTS / NWAVE>(p, pa, h, it, wave, lane, sPl, sMk, sPre, split, b, n_items, i0,
                                                      n, dense, writer, omk, Tb, nbb);
}

// The split pass of workgroup `bid` of the decode grid (attn_grid): NT threads. PLANNED (masked,
// unragged partition): the list is the plan's decision for (b, h), made in this workgroup's
// prologue from the scores pass's partials (pa): wavefront 0 decides (as plan_decide; every
// workgroup of the head reaches the same result from the same partials) and puts the chunk masks
// and their prefixes into LDS, from which all threads place this split's list positions; split 0 also stores trig, est and, at its end, the head's block
// list and count (the age is advanced by the update). With seq_lens (one sequence) its length
// comes from device memory; the grid is still num_splits x Hkv x B. With pa->pass_budget > 0 the
// prologue is planned_balanced's instead (grid pass_budget + B Hkv, num_splits partial slots).
template <int D, int G, bool MASKED, bool STATS, bool LOAD_V, bool MF, bool RAG, bool PLANNED = false,
          bool PAGED = false>
__device__ __forceinline__ void decode_body(const AttnP& p, int bid, const kvskip_plan_args* pa = nullptr) {
  static_assert(!PLANNED || MASKED, "a planned pass is masked");
  static_assert(!(PLANNED && RAG && PAGED), "a planned ragged pass reads a contiguous cache");
  static_assert(!PAGED || MF, "a paged cache is read by the MFMA engine");
  constexpr int GP = gpad<G>();
  __shared__ __attribute__((aligned(16))) float sP[NWAVE][BLK * GP];
  __shared__ __attribute__((aligned(16))) MergeLds<D, G> sL;

  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE;
  const int r8 = lane >> 3, sub = lane & 7;

  // This workgroup's work: (b, KV head h, split) and list positions / blocks [i0, i0 + n) of the
  // n_items of (b, h); Tb, nbb: the sequence's tokens and blocks.
  int split, h, b, n_items, i0, n;
  int Tb = p.T, nbb = p.nb;
  __shared__ int sPl[PLANNED ? MAX_NB + 1 : 1];  // planned: list positions i0 - 1 .. i0 + n - 1
  __shared__ int sPi[2];                          // planned: refresh, list length
  __shared__ uint32_t sMk[PLANNED ? MAX_NB / WCB : 1];  // planned: the list's chunk masks
  __shared__ int sPre[PLANNED ? MAX_NB / WCB : 1];      // planned: their exclusive prefixes
  uint32_t pmk[DCL];                              // planned, wavefront 0: the chunk masks
  bool dense = false;                             // planned: a refresh (every block, in order)
  const bool balanced = PLANNED && pa->pass_budget > 0;  // every list cut by one chunk length
  bool list_writer = false;                               // balanced: this wavefront writes the list
  // planned: the pass's partial slots [slot_base, slot_base + nslot) of the num_splits per head
  const int nslot = PLANNED && pa->slot_count > 0 ? pa->slot_count : p.num_splits;
  const int slot_base = PLANNED ? pa->slot_base : 0;
  // a refresh pass of the post-pass decision reads blocks whose neighbours' statistics the attended
  // pass wrote: it writes no gap statistics
  const bool gaps = !(PLANNED && pa->decide_mode == DECIDE_POST);
  if constexpr (PLANNED && RAG) {
    const int W = p.num_splits + p.B;
    const int it = xcd_remap(bid, W * p.Hkv);
    h = it / W;
    if (!planned_ragged<G>(p, *pa, h, it % W, wave, lane, sPl, sMk, sPre, split, b, n_items, i0, n, dense,
                           list_writer, pmk, Tb, nbb))
      return;
  } else if constexpr (PLANNED) {
    if (balanced) {
      if (p.seq_lens != nullptr) {  // one sequence whose length is in device memory
        Tb = seq_len(p, 0);
        nbb = (Tb + BLK - 1) / BLK;
      }
      if (!planned_balanced<G>(p, *pa, bid, wave, lane, nbb, sPl, sMk, sPre, split, h, b, n_items, i0, n, dense,
                               list_writer, pmk))
        return;
    } else {
      work_coords(bid, nslot, p.Hkv, p.B, split, h, b);
      if (p.seq_lens != nullptr) {  // one sequence whose length is in device memory
        Tb = seq_len(p, b);
        nbb = (Tb + BLK - 1) / BLK;
      }
      if (wave == 0) {
        int pre[DCL];
        const int mode = pa->decide_mode;
        const bool t = decide_head<G>(*pa, b, h, lane, pmk, split == 0 && mode != DECIDE_LISTS, false, mode, nbb);
        const int cnt = t ? nbb : mask_prefix(pmk, lane, plan_chunks(pa->T), pre);
        if (!t) {
#pragma unroll
          for (int d = 0; d < DCL; ++d) {
            sMk[lane + WAVE * d] = pmk[d];
            sPre[lane + WAVE * d] = pre[d];
          }
        }
        if (lane == 0) {
          sPi[0] = t ? 1 : 0;
          sPi[1] = cnt;
        }
      }
      __syncthreads();
      dense = sPi[0] != 0;
      n_items = sPi[1];
      const int per = (n_items + nslot - 1) / nslot;
      i0 = min(n_items, split * per);
      n = min(n_items, i0 + per) - i0;
      if (!dense) {  // this split's slice, positions i0 - 1 .. i0 + n - 1, by every thread
        slice_from_masks(sMk, sPre, plan_chunks(pa->T), i0, i0 + n, sPl, tid, NT);
        if (tid == 0 && i0 == 0) sPl[0] = -1;
        __syncthreads();
      }
    }
  } else if constexpr (!RAG) {
    work_coords(bid, p.num_splits, p.Hkv, p.B, split, h, b);
    n_items = MASKED ? min(max(p.block_cnt[b * p.Hkv + h], 0), p.max_blocks) : p.nb;
    const int per = (n_items + p.num_splits - 1) / p.num_splits;
    i0 = min(n_items, split * per);
    n = min(n_items, i0 + per) - i0;
  } else {  // ragged: ceil(n / C) chunks per list over the whole batch, per KV head or over all lists
    const int W = p.num_splits + p.B;
    const bool global = MASKED && p.list_partition != 0;
    // per KV head: a head's chunk slots on one XCD (its first slots are the busy ones on every XCD);
    // over all lists the busy chunks are the grid's first, so consecutive chunks go to consecutive
    // XCDs (remapped, the grid's idle tail left whole XCDs idle: B 32 at 64k, full lists, 1809 vs
    // 1385 us per pass)
    const int it = global ? bid : xcd_remap(bid, W * p.Hkv);
    int chunk, C;
    if (global) {
      C = global_lookup(p, it, b, h, chunk, n_items);
    } else {
      h = it / W;
      C = ragged_lookup(p, h, it % W, MASKED, b, chunk, n_items);
    }
    if constexpr (MASKED && STATS) {
      // (b', eh) with an empty list have no chunk: their statistics are written by one workgroup
      // per KV head eh (the head's first chunk slot; over all lists, workgroup eh)
      const int eh = global ? (it < p.Hkv ? it : -1) : (it % W == 0 ? h : -1);
      if (eh >= 0) {
        for (int b0 = wave * WAVE; b0 < p.B; b0 += NT) {
          const int bb = b0 + lane;
          uint64_t empty = __ballot(bb < p.B && ragged_items(p, bb, eh, true) == 0);
          while (empty != 0) {
            const int be = b0 + __ffsll(static_cast<unsigned long long>(empty)) - 1;
            empty &= empty - 1;
            const int64_t q0 = static_cast<int64_t>(be) * p.Hq + static_cast<int64_t>(eh) * G;
            for (int t = lane; t < G * p.nb; t += WAVE) {
              p.blk_max[(q0 + t / p.nb) * p.nb + t % p.nb] = NEG_INF;
              p.blk_sum[(q0 + t / p.nb) * p.nb + t % p.nb] = 0.f;
            }
          }
        }
      }
    }
    if (b < 0) return;
    split = chunk;
    // A list's ceil(n / C) chunks: of near-equal length (no chunk of a few items beside full ones:
    // B 8 172.9 -> 171.4 us per layer-step, config 5's dense pass 111.9 -> 111.3), or of C items
    // and a partial last over all lists of a queued grid (global_lookup's order takes the partial
    // chunks last) or of groups over 4 (config 5's loop 125.1 -> 126.6 cut near-equal).
    if (global && (G > 4 || grid_queued(p))) {
      i0 = chunk * C;
      n = min(n_items, i0 + C) - i0;
    } else {
      const int k = max(1, (n_items + C - 1) / C);
      i0 = chunk * n_items / k;
      n = (chunk + 1) * n_items / k - i0;
    }
    Tb = seq_len(p, b);
    nbb = (Tb + BLK - 1) / BLK;
  }
  const int* glist = MASKED && !PLANNED ? p.block_idx + static_cast<int64_t>(b * p.Hkv + h) * p.max_blocks : nullptr;
  // entry at list position pos (planned: pos in [i0 - 1, i0 + n), from LDS; a refresh lists every block)
  const auto list = [&](int pos) -> int {
    if constexpr (PLANNED)
      return dense ? pos : sPl[pos - i0 + 1];
    else
      return glist[pos];
  };
  // Paged cache: the page (and, with a list, the block) of each of this workgroup's items i0 + t,
  // t < n, gathered into LDS once, so the streaming loop reads them without a vector-memory wait.
  // Blocks outside the sequence and page ids outside [0, num_pages) become -1 (an empty block).
  __shared__ int sPg[PAGED ? MAX_NB : 1];
  __shared__ int sBk[PAGED && MASKED ? MAX_NB : 1];
  if constexpr (PAGED)
    gather_pages(p, b, n, nbb, [&](int t) { return MASKED ? list(i0 + t) : i0 + t; }, sPg, MASKED ? sBk : nullptr);
  // paged: item k of this wavefront (LDS slot wave + NWAVE k): its block and page
  auto paged_item = [&](int k, int& blk, int& pg) {
    const int t = wave + NWAVE * k;
    pg = __builtin_amdgcn_readfirstlane(sPg[t]);
    if constexpr (MASKED)
      blk = __builtin_amdgcn_readfirstlane(sBk[t]);
    else
      blk = i0 + t;
  };
  const int nw = n > wave ? (n - wave + NWAVE - 1) / NWAVE : 0;  // this wavefront's items
  int gap_prev = -1, gap_cur = 0;  // masked stats: the list entries around this lane's gap
  if constexpr (MASKED && STATS) {
    const int t = wave + NWAVE * lane;
    if (t < n) {
      gap_cur = list(i0 + t);
      gap_prev = i0 + t > 0 ? list(i0 + t - 1) : -1;
    }
  }

  const rsrc_t rk = make_rsrc(p.k + b * p.k_sb + h * p.k_sh, head_bytes(Tb, p.k_st, D));
  const rsrc_t rv = make_rsrc(p.v + b * p.v_sb + h * p.v_sh, LOAD_V ? head_bytes(Tb, p.v_st, D) : 0);
  const uint32_t voff = static_cast<uint32_t>((lane / Lay<D>::VLPR) * p.v_st * 2 + 16 * (lane % Lay<D>::VLPR));
  const int64_t hq0 = static_cast<int64_t>(b) * p.Hq + static_cast<int64_t>(h) * G;

  float acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
  float* sPw = sP[wave];

  // List entry of this wavefront's k-th item (k clamped to its items): a vector load whose value is
  // used two items later, so that waiting for it never waits for the block loads issued after it.
  auto entry_of = [&](int k) -> int { return MASKED ? list(i0 + wave + NWAVE * min(k, nw - 1)) : 0; };
  // Block of the k-th item from its entry; out-of-range entries read block 0 and are masked.
  auto block_of = [&](int e, int k) -> int {  // uniform over the wavefront
    const int blk = __builtin_amdgcn_readfirstlane(MASKED ? e : i0 + wave + NWAVE * k);
    return (blk >= 0 && blk < nbb) ? blk : -1;
  };
  auto accumulate = [&](const u32x4 (&vr)[Lay<D>::VN], const float (&alpha)[G]) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] *= alpha[g];
    pv_block<D, G>(acc, vr, sPw, lane);
    __builtin_amdgcn_wave_barrier();
  };

  float m[G], l[G];
  if constexpr (MF) {
    // ---- MFMA engine: K(j) and V(j) both prefetched one block ahead.
    constexpr int KS = MLay<D>::KS;
    constexpr int NI = G < 4 ? G : 4;               // score rows i in use per lane group
    const int j4 = lane >> 4, c16 = lane & 15;
    const uint32_t koffm = static_cast<uint32_t>(c16 * p.k_st * 2 + 16 * j4);
    // statistics and P of this (b, KV head) through buffer resources: one 32-bit offset per lane
    // (head 4 j4 + i: + i * row bytes), the block in the scalar offset
    const uint32_t nb4 = 4u * static_cast<uint32_t>(p.nb), tp2 = 2u * static_cast<uint32_t>(p.t_pad);
    const rsrc_t rs_max = make_rsrc(STATS ? p.blk_max + hq0 * p.nb : nullptr, STATS ? G * nb4 : 0);
    const rsrc_t rs_sum = make_rsrc(STATS ? p.blk_sum + hq0 * p.nb : nullptr, STATS ? G * nb4 : 0);
    const rsrc_t rs_p = make_rsrc(STATS && p.p_out != nullptr ? p.p_out + hq0 * p.t_pad : nullptr,
                                  STATS && p.p_out != nullptr ? G * tp2 : 0);
    const uint32_t v_stat = 4u * j4 * nb4, v_p = 4u * j4 * tp2 + 2u * c16;
    u32x4 qa[KS];
    load_q_mf<D, G>(qa, p, b, h, lane);
    float mr[4], lr[4];                             // running (m, l) of head 4 j4 + i
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      mr[i] = NEG_INF;
      lr[i] = 0.f;
    }
    // block blk's scores (tokens >= lim masked: lim = Tb, or 0 for an empty block), statistics and P
    auto process = [&](int blk, int lim, const u32x4 (&kr)[4][KS], float (&alpha)[G]) {
      const int t0 = blk >= 0 ? blk * BLK : 0;
      float s[4][4];
      qk_block_mf<D>(s, kr, qa, p.scale_log2, t0, lim, lane);
      float pv[4][4], ar[4];
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int g = 4 * j4 + i;
        const float mt = row16_max(fmaxf(fmaxf(s[0][i], s[1][i]), fmaxf(s[2][i], s[3][i])));
        const float mtu = mt == NEG_INF ? 0.f : mt;
        float e[4];
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) e[nt] = fexp2(s[nt][i] - mtu);
        const float st = row16_sum((e[0] + e[1]) + (e[2] + e[3]));
        const float m_new = fmaxf(mr[i], mt);
        const float mu = m_new == NEG_INF ? 0.f : m_new;
        ar[i] = fexp2(mr[i] - mu);
        const float cf = mt == NEG_INF ? 0.f : fexp2(mt - mu);
        lr[i] = lr[i] * ar[i] + st * cf;
        mr[i] = m_new;
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) pv[nt][i] = e[nt] * cf;
        if constexpr (STATS) {
          if (blk >= 0 && g < G) {
            if (c16 == 0) {
              bstore_f32(mt * LN2, rs_max, v_stat + i * nb4, 4 * blk);
              bstore_f32(st, rs_sum, v_stat + i * nb4, 4 * blk);
            }
            if (p.p_out != nullptr) {
#pragma unroll
              for (int nt = 0; nt < 4; ++nt) bstore_u16(f2h(e[nt]), rs_p, v_p + i * tp2 + 32 * nt, 2 * t0);
            }
          }
        }
      }
      if constexpr (LOAD_V) {
        if (4 * j4 < GP) {
#pragma unroll
          for (int nt = 0; nt < 4; ++nt)
            *reinterpret_cast<float4*>(sPw + (16 * nt + c16) * GP + 4 * j4) =
                make_float4(pv[nt][0], NI > 1 ? pv[nt][1] : 0.f, NI > 2 ? pv[nt][2] : 0.f, NI > 3 ? pv[nt][3] : 0.f);
        }
      }
#pragma unroll
      for (int g = 0; g < G; ++g) alpha[g] = lane_value(ar[g % 4], 16 * (g / 4));
    };
    if (nw > 0 && !LOAD_V && PAGED) {
      // K only over a paged cache: two blocks in flight as below, each through its page's resource
      u32x4 ka[4][KS], kb[4][KS];
      int b0, g0, b1 = -1, g1 = -1;
      paged_item(0, b0, g0);
      load_k_block_mf<D>(ka, block_rsrc(p.k, p.k_sb, p.k_sh, p.k_st, h, b0, g0, Tb, D), koffm, p.k_st,
                         max(b0, 0) * BLK);
      auto step = [&](u32x4 (&ld)[4][KS], int& bld, int& gld, const u32x4 (&ac)[4][KS], int bac, int gac, int k) {
        if (k + 1 < nw) {
          paged_item(k + 1, bld, gld);
        } else {
          bld = -1;
          gld = -1;
        }
        load_k_block_mf<D>(ld, block_rsrc(p.k, p.k_sb, p.k_sh, p.k_st, h, bld, gld, Tb, D), koffm, p.k_st,
                           max(bld, 0) * BLK);
        __builtin_amdgcn_sched_barrier(0);
        if (k < nw) {
          float alpha[G];
          process(bac, (bac >= 0 && gac >= 0) ? Tb : 0, ac, alpha);
        }
        __builtin_amdgcn_sched_barrier(0);
      };
      for (int k = 0; k < nw; k += 2) {
        step(kb, b1, g1, ka, b0, g0, k);
        step(ka, b0, g0, kb, b1, g1, k + 1);
      }
    } else if (nw > 0 && !LOAD_V) {
      // K only: two blocks in flight while one is scored (the V registers are free). Step k loads
      // item k + 1 and scores item k; past the last item the load reads beyond the head's buffer
      // range (zeros, no memory access), so every step issues the same loads.
      u32x4 ka[4][KS], kb[4][KS];
      int ea = entry_of(1), eb = entry_of(2);
      int b0 = block_of(entry_of(0), 0), b1 = -1;
      load_k_block_mf<D>(ka, rk, koffm, p.k_st, max(b0, 0) * BLK);
      auto step = [&](u32x4 (&ld)[4][KS], int& bld, const u32x4 (&ac)[4][KS], int bac, int k) {
        const int ec = entry_of(k + 3);
        bld = block_of(ea, min(k + 1, nw - 1));
        ea = eb;
        eb = ec;
        load_k_block_mf<D>(ld, rk, koffm, p.k_st, (k + 1 < nw ? max(bld, 0) : nbb) * BLK);
        __builtin_amdgcn_sched_barrier(0);
        if (k < nw) {
          float alpha[G];
          process(bac, bac >= 0 ? Tb : 0, ac, alpha);
        }
        __builtin_amdgcn_sched_barrier(0);
      };
      for (int k = 0; k < nw; k += 2) {
        step(kb, b1, ka, b0, k);
        step(ka, b0, kb, b1, k + 1);
      }
    } else if (nw > 0 && PAGED) {
      // each block's K / V resource spans its page's rows of this head that hold tokens (zeros
      // beyond), an empty block's spans nothing; both are built before the block ahead is scored
      // (built after it, the compiler spilled the freshly loaded K block)
      u32x4 kr[4][KS];
      u32x4 vr[Lay<D>::VN];
      auto page_rsrc = [&](const uint16_t* pool, int64_t psb, int64_t sh, int64_t st, int blk, int pg) {
        return block_rsrc(pool, psb, sh, st, h, blk, pg, Tb, D);
      };
      auto lim_of = [&](int blk, int pg) { return (blk >= 0 && pg >= 0) ? Tb : 0; };
      int blk, pg;
      paged_item(0, blk, pg);
      load_k_block_mf<D>(kr, page_rsrc(p.k, p.k_sb, p.k_sh, p.k_st, blk, pg), koffm, p.k_st, max(blk, 0) * BLK);
      load_v_block<D>(vr, page_rsrc(p.v, p.v_sb, p.v_sh, p.v_st, blk, pg), voff, p.v_st, max(blk, 0) * BLK);
      for (int k = 0; k + 1 < nw; ++k) {
        int blk_n, pg_n;
        paged_item(k + 1, blk_n, pg_n);
        const rsrc_t rk_n = page_rsrc(p.k, p.k_sb, p.k_sh, p.k_st, blk_n, pg_n);
        const rsrc_t rv_n = page_rsrc(p.v, p.v_sb, p.v_sh, p.v_st, blk_n, pg_n);
        float alpha[G];
        process(blk, lim_of(blk, pg), kr, alpha);
        __builtin_amdgcn_sched_barrier(0);
        load_k_block_mf<D>(kr, rk_n, koffm, p.k_st, max(blk_n, 0) * BLK);
        __builtin_amdgcn_sched_barrier(0);
        accumulate(vr, alpha);
        __builtin_amdgcn_sched_barrier(0);
        load_v_block<D>(vr, rv_n, voff, p.v_st, max(blk_n, 0) * BLK);
        blk = blk_n;
        pg = pg_n;
      }
      float alpha[G];
      process(blk, lim_of(blk, pg), kr, alpha);
      accumulate(vr, alpha);
    } else if (nw > 0) {
      u32x4 kr[4][KS];
      u32x4 vr[Lay<D>::VN];
      int e_n = entry_of(1);
      int blk = block_of(entry_of(0), 0);
      load_k_block_mf<D>(kr, rk, koffm, p.k_st, max(blk, 0) * BLK);
      if constexpr (LOAD_V) load_v_block<D>(vr, rv, voff, p.v_st, max(blk, 0) * BLK);
      for (int k = 0; k + 1 < nw; ++k) {
        const int e_nn = entry_of(k + 2);
        const int blk_n = block_of(e_n, k + 1);
        e_n = e_nn;
        float alpha[G];
        process(blk, blk >= 0 ? Tb : 0, kr, alpha);
        __builtin_amdgcn_sched_barrier(0);
        load_k_block_mf<D>(kr, rk, koffm, p.k_st, max(blk_n, 0) * BLK);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (LOAD_V) {
          accumulate(vr, alpha);
          __builtin_amdgcn_sched_barrier(0);
          load_v_block<D>(vr, rv, voff, p.v_st, max(blk_n, 0) * BLK);
        }
        blk = blk_n;
      }
      float alpha[G];
      process(blk, blk >= 0 ? Tb : 0, kr, alpha);
      if constexpr (LOAD_V) accumulate(vr, alpha);
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      m[g] = lane_value(mr[g % 4], 16 * (g / 4));
      l[g] = lane_value(lr[g % 4], 16 * (g / 4));
    }
  } else {
    // ---- VALU engine: V(j) issued after QK(j), together with K(j+1) (register budget).
    const uint32_t koff = static_cast<uint32_t>(r8 * p.k_st * 2 + 16 * sub);
    u32x4 qv[G][Lay<D>::KC];
    load_q<D, G>(qv, p, b, h, lane);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      m[g] = NEG_INF;
      l[g] = 0.f;
    }
    auto process = [&](int blk, const u32x4 (&kr)[8][Lay<D>::KC], float (&alpha)[G]) {
      const int t0 = blk >= 0 ? blk * BLK : 0;
      float s[8][G];
      qk_block<D, G>(s, kr, qv, p.scale_log2, t0, blk >= 0 ? Tb : 0, lane);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float e[8], mt, st, c;
        block_softmax<G>(s, g, m[g], l[g], e, mt, st, alpha[g], c);
        if constexpr (STATS) {
          if (blk >= 0) {
            const int64_t hq = hq0 + g;
            if (lane == 0) {
              p.blk_max[hq * p.nb + blk] = mt * LN2;
              p.blk_sum[hq * p.nb + blk] = st;
            }
            if (p.p_out != nullptr && sub == g) {
#pragma unroll
              for (int rg = 0; rg < 8; ++rg) p.p_out[hq * p.t_pad + t0 + 8 * rg + r8] = f2h(e[rg]);
            }
          }
        }
        if constexpr (LOAD_V) {
          if (sub == 0) {
#pragma unroll
            for (int rg = 0; rg < 8; ++rg) sPw[(8 * rg + r8) * GP + g] = e[rg] * c;
          }
        }
      }
    };
    if (nw > 0) {
      u32x4 kr[8][Lay<D>::KC];
      u32x4 vr[Lay<D>::VN];
      int e_n = entry_of(1);
      int blk = block_of(entry_of(0), 0);
      load_k_block<D>(kr, rk, koff, p.k_st, max(blk, 0) * BLK);
      for (int k = 0; k + 1 < nw; ++k) {
        const int e_nn = entry_of(k + 2);
        const int blk_n = block_of(e_n, k + 1);
        e_n = e_nn;
        float alpha[G];
        process(blk, kr, alpha);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (LOAD_V) load_v_block<D>(vr, rv, voff, p.v_st, max(blk, 0) * BLK);
        load_k_block<D>(kr, rk, koff, p.k_st, max(blk_n, 0) * BLK);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (LOAD_V) accumulate(vr, alpha);
        blk = blk_n;
      }
      float alpha[G];
      process(blk, kr, alpha);
      if constexpr (LOAD_V) {
        load_v_block<D>(vr, rv, voff, p.v_st, max(blk, 0) * BLK);
        accumulate(vr, alpha);
      }
    }
  }
  finish<D, G, LOAD_V>(p, m, l, acc, b, h, slot_base + split, sL, false);
  if constexpr (MASKED && STATS)
    if (gaps) write_gap_stats<G>(p, list, n_items, i0, n, split, hq0, wave, lane, gap_prev, gap_cur);
  if constexpr (PLANNED) {
    if ((balanced || RAG) ? list_writer : (split == 0 && wave == 0))
      write_block_list(*pa, static_cast<int64_t>(b) * p.Hkv + h, nbb, dense, pmk, lane);
  }
  if constexpr (!MASKED && STATS && RAG) {  // the blocks past the sequence's end read (-inf, 0)
    if (nbb < p.nb && i0 + n == n_items) {
      for (int t = tid; t < G * (p.nb - nbb); t += NT) {
        const int64_t i = (hq0 + t / (p.nb - nbb)) * p.nb + nbb + t % (p.nb - nbb);
        p.blk_max[i] = NEG_INF;
        p.blk_sum[i] = 0.f;
      }
    }
  }
}

}  // namespace
}  // namespace kvs
