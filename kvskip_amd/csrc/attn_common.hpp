// Shared device code of the split-K flash-decode kernels for gfx950 (attn_decode.hip: dense,
// block-list, per-block statistics, stats-only, fp16 P; attn_vskip.hip: single-pass V-skip,
// two-pass V-skip pass 2, read ceiling).
//
// Work decomposition. num_splits * Hkv * B workgroups of NWAVE wavefronts; a workgroup owns one
// contiguous range of "items" (64-token blocks, or entries of a block list) of one KV head
// and serves all G query heads of that head, so each K/V byte is read once. Workgroups are
// dispatched round-robin over the 8 XCDs; the launch index is remapped so that consecutive
// work items (the splits of one KV head) land on the same XCD.
// Inside the workgroup the wavefronts are independent streams: wavefront w takes items w,
// w+NWAVE, ... and keeps its own online-softmax state for the G heads, so the main loop has no
// workgroup barrier. A wavefront processes a whole 64-token block at a time, so the
// per-block statistics fall out of its own registers. The 4 states are merged once, in LDS,
// at the end. With num_splits > 1 each workgroup writes its partial state and a second,
// short kernel merges the splits (8 split classes x 32 dims per workgroup). A merge inside the
// same kernel (last-arriving workgroup) costs more than that launch on gfx950: with device-scope
// fences (an L2 write-back and invalidate per workgroup) 2x slower at 2 workgroups per CU; with
// the partials stored and read at agent scope (no write-back) and a self-resetting ticket, +3.8 us
// per op at config 2 (dense and masked alike, graph-replayed or eager): the pass's tail gains
// three dependent memory round trips (store completion, ticket, partials), more than the
// dispatch gap of the merge kernel.
//
// Pipeline per wavefront: K(j) and V(j) are in flight when block j starts; after QK(j) the K
// loads of block j+1 are issued, after PV(j) its V loads. The last block is peeled off the
// loop so every load in the loop is unconditional (exact wait counts).
//
// QK runs on one of two engines (chosen per launch, KVSKIP_AMD_QK=valu|mfma):
//   mfma  v_mfma_f32_16x16x32_bf16 with the G query heads as the 16 M rows (zero-padded), 16
//         tokens as N and 32 dims as K: Q is 4 VGPRs per 32 dims whatever G, a 64-token block
//         is 4 x (D/32) MFMAs, and the scores come out as lane (j = lane/16, c = lane%16)
//         holding heads 4j..4j+3 of token c of each 16-token tile; block max / sum are 4-step
//         DPP reductions inside the 16-lane row.
//   valu  (below) dot products on v_dot2_f32_bf16.
// Lane layouts (64 lanes, D = 64 or 128):
//   K   8 lanes per token row, 8 rows per load; lane (r8 = lane/8, sub = lane%8) holds rows
//       8*rg + r8 (rg = 0..7), dims [8 sub, 8 sub + 8) (+64 for D = 128), as packed bf16.
//       QK = v_dot2_f32_bf16 against the unscaled bf16 query (exact products, fp32 sums),
//       then a 3-step DPP sum over the 8 lanes of the row; the score is scaled after.
//   V   D/8 lanes per row, 8 dims per lane, 16-byte loads; lane accumulates its rows for
//       all G heads in fp32 (acc[G][8]); P reaches the V layout through a per-wavefront
//       LDS tile [64][G] written after the softmax.
// Softmax runs in log2 units (v_exp_f32); per head and block: block max mt, e = 2^(s - mt)
// (the block statistics), p = e * 2^(mt - m_run). K/V are read through buffer resources
// bounded to the head's rows, so rows past T read as zeros; their scores are masked to -inf.
#pragma once

#include "common.hpp"
#include "internal.hpp"

namespace kvs {
namespace {

#ifndef KVS_NWAVE
#define KVS_NWAVE 4
#endif
constexpr int NWAVE = KVS_NWAVE;  // wavefronts per attention workgroup
constexpr int NT = NWAVE * WAVE;

template <int D>
struct Lay {
  static_assert(D == 64 || D == 128, "head dim");
  static constexpr int KC = D / 64;         // 16-byte K chunks per lane per row
  static constexpr int VLPR = D / 8;        // lanes per V row
  static constexpr int VRPI = WAVE / VLPR;  // V rows per load instruction
  static constexpr int VN = BLK / VRPI;     // V load instructions per block
};

template <int G>
constexpr int gpad() {
  return G <= 4 ? 4 : 8;
}

// Launch index -> work index, XCD-aware when n % 8 == 0: launch index i is dispatched to XCD
// i % 8, and w = (i % 8) * (n / 8) + i / 8 gives each XCD a contiguous run of work items (a
// launch whose first workgroups do other work only rotates which XCD holds which run).
__device__ __forceinline__ int xcd_remap(int i, int n) { return n % 8 == 0 ? (i % 8) * (n / 8) + i / 8 : i; }

// Work coordinates (split, KV head, sequence) of decode workgroup `bid`.
__device__ __forceinline__ void work_coords(int bid, int S, int Hkv, int B, int& split, int& h, int& b) {
  const int i = xcd_remap(bid, S * Hkv * B);
  split = i % S;
  const int r = i / S;
  h = r % Hkv;
  b = r / Hkv;
}
__device__ __forceinline__ void work_coords(int S, int Hkv, int B, int& split, int& h, int& b) {
  work_coords(blockIdx.x, S, Hkv, B, split, h, b);
}

// ---- Ragged batches (seq_lens): sequence b attends tokens [0, clamp(seq_lens[b], 1, T)).
__device__ __forceinline__ int seq_len(const AttnP& p, int b) {
  return p.seq_lens != nullptr ? min(max(p.seq_lens[b], 1), p.T) : p.T;
}

// Items of sequence b on KV head h: its blocks (dense) or its list entries (masked).
__device__ __forceinline__ int ragged_items(const AttnP& p, int b, int h, bool masked) {
  if (masked) return min(max(p.block_cnt[b * p.Hkv + h], 0), p.max_blocks);
  return (seq_len(p, b) + BLK - 1) / BLK;
}

// Chunk lengths of the ragged partitions. A length C0 set for S slots of a (S + B)-slot grid
// (S = num_splits) leaves the grid's last B slots to the sequences' (or lists') partial chunks, so
// where the whole grid is resident (at most RESIDENT_SLOTS workgroups: two per CU) most CUs hold
// full chunks and the rest partial ones. There, with long chunks (C0 >= 32 items), C is the smallest
// length whose chunks (sum of ceil(n / C) over the lanes' counts nv) still fit the slots, found by
// bisection between lo and C0 (C0 fits), and at least lo; with short chunks or a queued grid the
// shorter chunks' fixed costs win. Config 5's dense pass (per-head partition, one workgroup per CU):
// 121.0 -> 113.2 us per layer-step. Uniform.
constexpr int RESIDENT_SLOTS = 512;

// A ragged grid ((num_splits + B) * Hkv workgroups) longer than the resident slots: its queued
// workgroups start as others end.
__device__ __forceinline__ bool grid_queued(const AttnP& p) {
  return (p.num_splits + p.B) * p.Hkv > RESIDENT_SLOTS;
}

template <int NR>
__device__ __forceinline__ int fit_chunk_len(const AttnP& p, const int (&nv)[NR], int n_lists, int lo, int c0,
                                             int slots) {
  if (grid_queued(p) || c0 < 32) return c0;
  int hi = c0;
  lo = __builtin_amdgcn_readfirstlane(min(lo, c0));
  while (lo < hi) {  // the chunk count does not grow with C
    const int mid = (lo + hi) >> 1;
    int n = 0;
#pragma unroll
    for (int r = 0; r < NR; ++r)
      if (r * WAVE < n_lists) n += (nv[r] + mid - 1) / mid;
    n = __builtin_amdgcn_readfirstlane(wave_sum_int(n));
    if (n <= slots)
      hi = mid;
    else
      lo = mid + 1;
  }
  return lo;
}

// Ragged partition of KV head h (per head; list_partition 0): the items of its B sequences (blocks,
// or list entries when masked) in chunks of one length C, numbered sequence by sequence, at most
// S + B chunks per head (C0 = ceil(sum_b items_b / S); bisected as fit_chunk_len says, at least
// ceil(most / S) so that no sequence has more than S chunks). Lane j holds sequences j + 64 r in nv.
// Returns C, uniform.
constexpr int NRB = MAX_RAGGED_B / WAVE;

__device__ __forceinline__ int ragged_chunk_len(const AttnP& p, int h, bool masked, int (&nv)[NRB]) {
  const int lane = threadIdx.x % WAVE;
  int tot = 0, most = 0;
#pragma unroll
  for (int r = 0; r < NRB; ++r) {
    const int bb = r * WAVE + lane;
    nv[r] = bb < p.B ? ragged_items(p, bb, h, masked) : 0;
    tot += nv[r];
    most = max(most, nv[r]);
  }
  tot = wave_sum_int(tot);
  most = static_cast<int>(wave_max(static_cast<float>(most)));  // exact: counts <= 2^24
  const int S = p.num_splits;
  const int c0 = __builtin_amdgcn_readfirstlane(max(1, (tot + S - 1) / S));
  const int lo = max(max(1, (most + S - 1) / S), (tot + S + p.B - 1) / (S + p.B));
  return fit_chunk_len(p, nv, p.B, lo, c0, S + p.B);
}

// Chunk number `it` of KV head h's ragged partition, uniform over the wavefront: b (-1 past the
// head's last chunk), the chunk within b and b's item count. Returns C.
__device__ int ragged_lookup(const AttnP& p, int h, int it, bool masked, int& b, int& chunk, int& items) {
  const int lane = threadIdx.x % WAVE;
  int nv[NRB];
  const int C = ragged_chunk_len(p, h, masked, nv);
  b = -1;
  chunk = 0;
  items = 0;
  int base = 0;
#pragma unroll
  for (int r = 0; r < NRB; ++r) {
    if (r * WAVE >= p.B) break;
    const int ch = (nv[r] + C - 1) / C;
    const int incl = wave_incl_scan(ch);
    const int excl = base + incl - ch;
    const uint64_t hit = __ballot(ch > 0 && it >= excl && it < excl + ch);
    if (hit != 0) {
      const int l = __ffsll(static_cast<unsigned long long>(hit)) - 1;
      b = r * WAVE + l;
      chunk = it - __shfl(excl, l, WAVE);
      items = __shfl(nv[r], l, WAVE);
    }
    base += __shfl(incl, WAVE - 1, WAVE);
  }
  b = __builtin_amdgcn_readfirstlane(b);  // uniform: scalar registers for the addressing that follows
  chunk = __builtin_amdgcn_readfirstlane(chunk);
  items = __builtin_amdgcn_readfirstlane(items);
  return C;
}

// Chunks (split partials) of (b, KV head h) under the ragged partition.
__device__ __forceinline__ int ragged_chunks(const AttnP& p, int b, int h, bool masked) {
  int nv[NRB];
  const int C = ragged_chunk_len(p, h, masked, nv);
  return (ragged_items(p, b, h, masked) + C - 1) / C;
}

// Partition over all B * Hkv lists of a masked ragged pass (p.list_partition = 1): ceil(n / C)
// chunks of each list's n entries (their bounds: decode_body), numbered list by list (l = b Hkv +
// h), so a KV head whose lists hold more entries (a refreshing sequence) gets more workgroups
// instead of longer chunks. C0 = max(ceil(sum /
// (S Hkv)), ceil(most / S)) fits the grid's (S + B) Hkv slots (sum / C0 <= S Hkv, plus at most one
// partial chunk per list), bisected as fit_chunk_len says (per layer-step with carried updates,
// config 5 131.1 -> 125.0 us, B 8 179.1 -> 173.4; bisected for every grid, B 8 with stable queries
// +0.4 us and B 32 at 64k +3.5 us). Lane j holds lists j + 64 r in nv. Returns C, uniform.
constexpr int NRG = MAX_GLOBAL_LISTS / WAVE;

__device__ __forceinline__ int global_chunk_len(const AttnP& p, int (&nv)[NRG]) {
  const int lane = threadIdx.x % WAVE, nl = p.B * p.Hkv;
  int tot = 0, most = 0;
#pragma unroll
  for (int r = 0; r < NRG; ++r) {
    const int l = r * WAVE + lane;
    nv[r] = l < nl ? min(max(p.block_cnt[l], 0), p.max_blocks) : 0;
    tot += nv[r];
    most = max(most, nv[r]);
  }
  tot = wave_sum_int(tot);
  most = static_cast<int>(wave_max(static_cast<float>(most)));  // exact: counts <= 2^24
  const int S = p.num_splits, slots = (S + p.B) * p.Hkv;
  const int c_min = max(1, (most + S - 1) / S);
  const int c0 = __builtin_amdgcn_readfirstlane(max(c_min, (tot + S * p.Hkv - 1) / (S * p.Hkv)));
  return fit_chunk_len(p, nv, nl, max(c_min, (tot + slots - 1) / slots), c0, slots);
}

// Chunk number `it` of the partition over all lists: its list (b, h; b = -1 past the last chunk),
// the chunk within the list and the list's entry count. Returns C. Uniform results. A grid longer
// than the resident slots (queued workgroups start as others end) takes the lists' full chunks
// first and their partial last chunks after them, the longer half of those first, so that it ends
// on its shortest chunks (B 32 at 64k, stable queries: 592.4 -> 579.8 us per layer-step, and
// 580.2-582.0 -> 577.6-578.1 with the two classes of partial chunks); a resident grid takes them
// list by list.
__device__ int global_lookup(const AttnP& p, int it, int& b, int& h, int& chunk, int& items) {
  const int lane = threadIdx.x % WAVE, nl = p.B * p.Hkv;
  int nv[NRG];
  const int C = global_chunk_len(p, nv);
  const bool queued = grid_queued(p);
  int l_sel = -1;
  chunk = 0;
  items = 0;
  int base = 0;
  // round one: every chunk of a list (resident grid) or its full chunks (queued grid)
#pragma unroll
  for (int r = 0; r < NRG; ++r) {
    if (r * WAVE >= nl) break;
    const int ch = queued ? nv[r] / C : (nv[r] + C - 1) / C;
    const int incl = wave_incl_scan(ch);
    const int excl = base + incl - ch;
    const uint64_t hit = __ballot(ch > 0 && it >= excl && it < excl + ch);
    if (hit != 0) {
      const int j = __ffsll(static_cast<unsigned long long>(hit)) - 1;
      l_sel = r * WAVE + j;
      chunk = it - __shfl(excl, j, WAVE);
      items = __shfl(nv[r], j, WAVE);
    }
    base += __shfl(incl, WAVE - 1, WAVE);
  }
  // rounds two and three: the partial last chunks, the longer ones (at least C / 2) first
  for (int cls = 0; cls < 2 && queued && __builtin_amdgcn_readfirstlane(l_sel) < 0; ++cls) {
#pragma unroll
    for (int r = 0; r < NRG; ++r) {
      if (r * WAVE >= nl) break;
      const int rem = nv[r] % C;
      const int part = rem != 0 && (2 * rem >= C) == (cls == 0) ? 1 : 0;
      const int incl = wave_incl_scan(part);
      const uint64_t hit = __ballot(part != 0 && it == base + incl - 1);
      if (hit != 0) {
        const int j = __ffsll(static_cast<unsigned long long>(hit)) - 1;
        l_sel = r * WAVE + j;
        items = __shfl(nv[r], j, WAVE);
        chunk = items / C;
      }
      base += __shfl(incl, WAVE - 1, WAVE);
    }
  }
  l_sel = __builtin_amdgcn_readfirstlane(l_sel);
  b = l_sel >= 0 ? l_sel / p.Hkv : -1;
  h = l_sel >= 0 ? l_sel % p.Hkv : 0;
  chunk = __builtin_amdgcn_readfirstlane(chunk);
  items = __builtin_amdgcn_readfirstlane(items);
  return C;
}

// Byte range of one (b, head) of a K or V view: rows 0..T-1 of D bf16 each, row stride st.
__device__ __forceinline__ uint32_t head_bytes(int T, int64_t st, int D) {
  return static_cast<uint32_t>((static_cast<int64_t>(T - 1) * st + D) * 2);
}

// ---- Paged cache: block blk of a sequence's KV head h is page pg of a pool (page stride psb
// elements, head stride sh, row stride st). The resource's base is placed 64 blk rows before the
// page, so the block's loads use the offsets of a view (token t0 = 64 blk); its range ends at the
// block's last token below Tb (rows past it read zero) and is empty for an empty block (blk or pg
// < 0). No offset below the page is ever formed.
__device__ __forceinline__ rsrc_t block_rsrc(const uint16_t* pool, int64_t psb, int64_t sh, int64_t st, int h,
                                             int blk, int pg, int Tb, int D) {
  if (blk < 0 || pg < 0) return make_rsrc(pool, 0u);
  return make_rsrc(pool + static_cast<int64_t>(pg) * psb + static_cast<int64_t>(h) * sh -
                       static_cast<int64_t>(blk) * BLK * st,
                   head_bytes(min(Tb, blk * BLK + BLK), st, D));
}

// The pages of a workgroup's items t < n (block blk_of(t)) of sequence b into LDS sPg (and the
// blocks into sBk, if given): -1 for blocks outside [0, nb) and page ids outside [0, num_pages).
// One pass of the workgroup's threads, then a barrier; the streaming loops read these without a
// vector-memory wait.
template <class BlockOf>
__device__ __forceinline__ void gather_pages(const AttnP& p, int b, int n, int nb, BlockOf blk_of, int* sPg,
                                             int* sBk) {
  const int* tbl = p.block_table + static_cast<int64_t>(b) * p.bt_stride;
  for (int t = threadIdx.x; t < n; t += blockDim.x) {
    int blk = blk_of(t);
    if (blk < 0 || blk >= nb) blk = -1;
    int pg = blk >= 0 ? tbl[blk] : -1;
    if (pg < 0 || pg >= p.num_pages) pg = -1;
    sPg[t] = pg;
    if (sBk != nullptr) sBk[t] = blk;
  }
  __syncthreads();
}

// K block at token t0: lane (r8, sub) gets rows t0 + 8 rg + r8, 16-byte chunks sub (+8).
// koff = r8 * k_st * 2 + 16 * sub (per lane, fixed).
template <int D>
__device__ __forceinline__ void load_k_block(u32x4 (&kr)[8][Lay<D>::KC], rsrc_t rk, uint32_t koff, int64_t k_st,
                                             int t0) {
  const uint32_t rowb = static_cast<uint32_t>(k_st * 2);
#pragma unroll
  for (int rg = 0; rg < 8; ++rg) {
    const uint32_t so = static_cast<uint32_t>(t0 + 8 * rg) * rowb;
#pragma unroll
    for (int c = 0; c < Lay<D>::KC; ++c) kr[rg][c] = bload16<BUF_NT>(rk, koff + 128 * c, so);
  }
}

// V block at token t0: lane (vrow, vsub) gets rows t0 + VRPI i + vrow, dims 8 vsub .. +8.
// voff = vrow * v_st * 2 + 16 * vsub.
template <int D>
__device__ __forceinline__ void load_v_block(u32x4 (&vr)[Lay<D>::VN], rsrc_t rv, uint32_t voff, int64_t v_st,
                                             int t0) {
  constexpr int VRPI = Lay<D>::VRPI;
  const uint32_t rowb = static_cast<uint32_t>(v_st * 2);
#pragma unroll
  for (int i = 0; i < Lay<D>::VN; ++i)
    vr[i] = bload16<BUF_NT>(rv, voff, static_cast<uint32_t>(t0 + VRPI * i) * rowb);
}

// Scores of one block in log2 units: s[rg][g] for row 8*rg + lane/8; rows t0 + r >= t_lim are
// masked to -inf (t_lim = T, or 0 for an invalid list entry).
template <int D, int G>
__device__ __forceinline__ void qk_block(float (&s)[8][G], const u32x4 (&kr)[8][Lay<D>::KC],
                                         const u32x4 (&qv)[G][Lay<D>::KC], float scale_log2, int t0, int t_lim,
                                         int lane) {
#pragma unroll
  for (int rg = 0; rg < 8; ++rg)
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float a = 0.f;
#pragma unroll
      for (int c = 0; c < Lay<D>::KC; ++c) a = dot8(qv[g][c], kr[rg][c], a);
      s[rg][g] = a;
    }
#pragma unroll
  for (int rg = 0; rg < 8; ++rg)
#pragma unroll
    for (int g = 0; g < G; ++g) s[rg][g] = sum8(s[rg][g]);
  const int r8 = lane >> 3;
#pragma unroll
  for (int rg = 0; rg < 8; ++rg) {
    const bool ok = t0 + 8 * rg + r8 < t_lim;
#pragma unroll
    for (int g = 0; g < G; ++g) s[rg][g] = ok ? s[rg][g] * scale_log2 : NEG_INF;
  }
}

// acc[g][e] += sum over the block's rows of P[row][g] * V[row][dims of this lane].
template <int D, int G>
__device__ __forceinline__ void pv_block(float (&acc)[G][8], const u32x4 (&vr)[Lay<D>::VN], const float* sPw,
                                         int lane) {
  constexpr int GP = gpad<G>();
  constexpr int VRPI = Lay<D>::VRPI;
  const int vrow = lane / Lay<D>::VLPR;
#pragma unroll
  for (int i = 0; i < Lay<D>::VN; ++i) {
    const float* pr = sPw + (VRPI * i + vrow) * GP;
    float pg[GP];
#pragma unroll
    for (int u = 0; u < GP; u += 4) {
      const float4 t = *reinterpret_cast<const float4*>(pr + u);
      pg[u] = t.x;
      pg[u + 1] = t.y;
      pg[u + 2] = t.z;
      pg[u + 3] = t.w;
    }
    float vf[8];
    vf[0] = bf_lo(vr[i].x);
    vf[1] = bf_hi(vr[i].x);
    vf[2] = bf_lo(vr[i].y);
    vf[3] = bf_hi(vr[i].y);
    vf[4] = bf_lo(vr[i].z);
    vf[5] = bf_hi(vr[i].z);
    vf[6] = bf_lo(vr[i].w);
    vf[7] = bf_hi(vr[i].w);
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] = fmaf(pg[g], vf[e], acc[g][e]);
  }
}

// Sum acc over the lanes that hold the same dims (the V row slots).
template <int D, int G>
__device__ __forceinline__ void reduce_acc_rows(float (&acc)[G][8]) {
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float a = acc[g][e];
      if constexpr (D == 64) a += dpp<DPP_ROR8>(a);
      a += xshfl(a, 16);
      a += xshfl(a, 32);
      acc[g][e] = a;
    }
}

// LDS of the workgroup epilogue.
template <int D, int G>
struct MergeLds {
  float acc[NWAVE * G * D];            // per-wavefront accumulators
  float ml[NWAVE * G * 2];             // per-wavefront (m, l)
};

// Workgroup epilogue: merge the wavefront states (m, l in log2 units, acc un-normalised), then
// write out/out_f32/lse (one split) or the split partials.
template <int D, int G, bool LOAD_V>
__device__ __forceinline__ void finish(const AttnP& p, float (&m)[G], float (&l)[G], float (&acc)[G][8], int b,
                                       int h, int split, MergeLds<D, G>& L, bool plain) {
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE;
  constexpr int VLPR = Lay<D>::VLPR;
  if constexpr (LOAD_V) {
    reduce_acc_rows<D, G>(acc);
    if (lane < VLPR) {
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) L.acc[(wave * G + g) * D + 8 * lane + e] = acc[g][e];
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      L.ml[(wave * G + g) * 2] = m[g];
      L.ml[(wave * G + g) * 2 + 1] = l[g];
    }
  }
  __syncthreads();
  const int S = p.num_splits;
  const int64_t hq0 = static_cast<int64_t>(b) * p.Hq + static_cast<int64_t>(h) * G;
  if constexpr (LOAD_V) {
    for (int o = tid; o < G * D; o += NT) {
      const int g = o / D, d = o % D;
      float A = 0.f, Ls = 0.f;
      if (plain) {
#pragma unroll
        for (int w = 0; w < NWAVE; ++w) A += L.acc[(w * G + g) * D + d];
        Ls = 1.f;
      } else {
        float M = NEG_INF;
#pragma unroll
        for (int w = 0; w < NWAVE; ++w) M = fmaxf(M, L.ml[(w * G + g) * 2]);
        const float mu = M == NEG_INF ? 0.f : M;
#pragma unroll
        for (int w = 0; w < NWAVE; ++w) {
          const float f = fexp2(L.ml[(w * G + g) * 2] - mu);
          Ls += L.ml[(w * G + g) * 2 + 1] * f;
          A += L.acc[(w * G + g) * D + d] * f;
        }
      }
      const int64_t hq = hq0 + g;
      if (S == 1) {
        const float o_ = Ls > 0.f ? A / Ls : 0.f;
        p.out[hq * D + d] = f2bf(o_);
        if (p.out_f32) p.out_f32[hq * D + d] = o_;
      } else {
        p.part_acc[(hq * S + split) * D + d] = A;
      }
    }
  }
  if (!plain && tid < G) {
    const int g = tid;
    float M = NEG_INF, Ls = 0.f;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) M = fmaxf(M, L.ml[(w * G + g) * 2]);
    const float mu = M == NEG_INF ? 0.f : M;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) Ls += L.ml[(w * G + g) * 2 + 1] * fexp2(L.ml[(w * G + g) * 2] - mu);
    const int64_t hq = hq0 + g;
    if (S == 1) {
      if (p.lse) p.lse[hq] = Ls > 0.f ? (M + flog2(Ls)) * LN2 : NEG_INF;
    } else {
      p.part_ml[(hq * S + split) * 2] = M;
      p.part_ml[(hq * S + split) * 2 + 1] = Ls;
    }
  }
}

template <int D, int G>
__device__ __forceinline__ void load_q(u32x4 (&qv)[G][Lay<D>::KC], const AttnP& p, int b, int h, int lane) {
  const int sub = lane & 7;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const uint16_t* qp = p.q + b * p.q_sb + (static_cast<int64_t>(h) * G + g) * p.q_sh + 8 * sub;
#pragma unroll
    for (int c = 0; c < Lay<D>::KC; ++c) qv[g][c] = ld16(qp + 64 * c);
  }
}

// One block's softmax step for head g: updates (m, l), returns alpha (rescale of acc) and the
// factor c with p = e * c; e = 2^(s - mt) and the block stats (mt, st) are left for the caller.
template <int G>
__device__ __forceinline__ void block_softmax(const float (&s)[8][G], int g, float& m, float& l, float (&e)[8],
                                              float& mt, float& st, float& alpha, float& c) {
  float x = s[0][g];
#pragma unroll
  for (int rg = 1; rg < 8; ++rg) x = fmaxf(x, s[rg][g]);
  mt = max_rows8(x);
  const float mtu = mt == NEG_INF ? 0.f : mt;
  float sum = 0.f;
#pragma unroll
  for (int rg = 0; rg < 8; ++rg) {
    e[rg] = fexp2(s[rg][g] - mtu);
    sum += e[rg];
  }
  st = sum_rows8(sum);
  const float m_new = fmaxf(m, mt);
  const float mu = m_new == NEG_INF ? 0.f : m_new;
  alpha = fexp2(m - mu);
  c = mt == NEG_INF ? 0.f : fexp2(mt - mu);
  l = l * alpha + st * c;
  m = m_new;
}


// ---------------------------------------------------------------- MFMA QK engine
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <int D>
struct MLay {
  static constexpr int KS = D / 32;  // 32-dim k-steps of v_mfma_f32_16x16x32_bf16
};

// Sum / max over the 16 lanes of each DPP row (every lane gets the row result).
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<DPP_XOR1>(v);
  v += dpp<DPP_XOR2>(v);
  v += dpp<DPP_HALF_MIRROR>(v);
  return v + dpp<DPP_MIRROR>(v);
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp<DPP_XOR1>(v));
  v = fmaxf(v, dpp<DPP_XOR2>(v));
  v = fmaxf(v, dpp<DPP_HALF_MIRROR>(v));
  return fmaxf(v, dpp<DPP_MIRROR>(v));
}

// B operand (K^T) of one 64-token block: kr[nt][kk] = 16 bytes of row t0 + 16 nt + lane%16 at
// 16-byte chunk 4 kk + lane/16. koffm = (lane % 16) * k_st * 2 + 16 * (lane / 16).
template <int D>
__device__ __forceinline__ void load_k_block_mf(u32x4 (&kr)[4][MLay<D>::KS], rsrc_t rk, uint32_t koffm,
                                                int64_t k_st, int t0) {
  const uint32_t rowb = static_cast<uint32_t>(k_st * 2);
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const uint32_t so = static_cast<uint32_t>(t0 + 16 * nt) * rowb;
#pragma unroll
    for (int kk = 0; kk < MLay<D>::KS; ++kk) kr[nt][kk] = bload16<BUF_NT>(rk, koffm + 64 * kk, so);
  }
}

// A operand (Q): lane (j, c = lane%16) holds head c's dims of chunk 4 kk + j (zero for c >= G).
template <int D, int G>
__device__ __forceinline__ void load_q_mf(u32x4 (&qa)[MLay<D>::KS], const AttnP& p, int b, int h, int lane) {
  const int c = lane & 15, j = lane >> 4;
  const uint16_t* qp = p.q + b * p.q_sb + (static_cast<int64_t>(h) * G + c) * p.q_sh + 8 * j;
#pragma unroll
  for (int kk = 0; kk < MLay<D>::KS; ++kk) qa[kk] = c < G ? ld16(qp + 32 * kk) : u32x4{0u, 0u, 0u, 0u};
}

// Scores of one block in log2 units, MFMA layout: s[nt][i] = head 4*(lane/16) + i, token
// t0 + 16 nt + lane%16; tokens >= t_lim masked to -inf.
template <int D>
__device__ __forceinline__ void qk_block_mf(float (&s)[4][4], const u32x4 (&kr)[4][MLay<D>::KS],
                                            const u32x4 (&qa)[MLay<D>::KS], float scale_log2, int t0, int t_lim,
                                            int lane) {
  const int c = lane & 15;
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    f32x4_t a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < MLay<D>::KS; ++kk)
      a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, qa[kk]),
                                                  __builtin_bit_cast(bf16x8_t, kr[nt][kk]), a, 0, 0, 0);
    const bool ok = t0 + 16 * nt + c < t_lim;
#pragma unroll
    for (int i = 0; i < 4; ++i) s[nt][i] = ok ? a[i] * scale_log2 : NEG_INF;
  }
}

// Split merge: workgroup (b*Hq + hq, 32-dim slice), 256 threads = 8 split classes x 32 dims.
// Thread (cls, d) loads the partials of splits s = cls + 8 u, u < U (U = ceil(S / 8), a template
// parameter so every load is unconditional, clamped to S - 1, and in flight together), the
// classes agree on the max through LDS, then weight (2^(m_s - M), log-sum-exp mode; 1, plain
// mode for the two-pass pass 2) and add in LDS. WITH_V = false (stats-only): only lse.
// Body of one merge workgroup (query head hq, dims [32 slice, 32 slice + 32)) over its Sv <= 8 U
// partials. A workgroup wider than 256 threads (the fused merge + update launch) runs it with its
// first 256; the others only pass the barriers.
template <int D, int U, bool WITH_V>
__device__ __forceinline__ void merge_body(const AttnP& p, int plain, int64_t hq, int slice, int Sv) {
  constexpr int NC = 8;
  const int tid = threadIdx.x, cls = (tid / 32) % NC, dl = tid % 32;
  const bool act = tid < 256;
  const int d = slice * 32 + dl;
  const int S = p.num_splits;
  const float* ml = p.part_ml + hq * S * 2;
  __shared__ float rA[NC][32], rL[NC], rM[NC];
  float ms[U], ls[U], as[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int s = max(min(cls + NC * u, Sv - 1), 0);
    const float2 t = *reinterpret_cast<const float2*>(ml + 2 * s);
    ms[u] = t.x;
    ls[u] = t.y;
    if constexpr (WITH_V) as[u] = p.part_acc[(hq * S + s) * D + d];
  }
  float mloc = NEG_INF;
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (cls + NC * u < Sv) mloc = fmaxf(mloc, ms[u]);
  if (act && dl == 0) rM[cls] = mloc;
  __syncthreads();
  float M = NEG_INF;
#pragma unroll
  for (int c = 0; c < NC; ++c) M = fmaxf(M, rM[c]);
  const float mu = M == NEG_INF ? 0.f : M;
  float A = 0.f, L = 0.f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (cls + NC * u < Sv && (plain || ls[u] > 0.f)) {  // an empty partial (l = 0) adds nothing
      const float w = plain ? 1.f : fexp2(ms[u] - mu);
      L += ls[u] * w;
      if constexpr (WITH_V) A += as[u] * w;
    }
  }
  if (act) rA[cls][dl] = A;
  if (act && dl == 0) rL[cls] = L;
  __syncthreads();
  if (tid < 32) {
    float a = 0.f, l = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      a += rA[c][tid];
      l += rL[c];
    }
    if (plain) l = 1.f;
    if constexpr (WITH_V) {
      const float o = l > 0.f ? a / l : 0.f;
      p.out[hq * D + d] = f2bf(o);
      if (p.out_f32) p.out_f32[hq * D + d] = o;
    }
    if (!plain && tid == 0 && slice == 0 && p.lse) p.lse[hq] = l > 0.f ? (M + flog2(l)) * LN2 : NEG_INF;
  }
}

// Partials of query head hq: S, or in a ragged batch its (sequence, KV head)'s chunk count (0:
// nothing attended, out 0 and lse -inf). Uniform over the workgroup.
__device__ __forceinline__ int merge_count(const AttnP& p, int64_t hq) {
  if (p.seq_lens == nullptr) return p.num_splits;
  const int b = static_cast<int>(hq / p.Hq), h = static_cast<int>(hq % p.Hq) / (p.Hq / p.Hkv);
  if (p.block_idx != nullptr && p.list_partition != 0) {
    int nv[NRG];
    const int C = global_chunk_len(p, nv);
    return (ragged_items(p, b, h, true) + C - 1) / C;
  }
  return ragged_chunks(p, b, h, p.block_idx != nullptr);
}

// merge_body with the fewest slots that hold Sv partials (U halved while 4 U still does): a ragged
// head with few chunks issues no loads for slots it does not have (at S = 128 most heads have a
// handful of chunks). Sv is uniform, so the choice is a uniform branch.
template <int D, int U, bool WITH_V>
__device__ void merge_fit(const AttnP& p, int plain, int64_t hq, int slice, int Sv) {
  if constexpr (U > 1) {
    if (Sv <= 8 * (U / 2)) {
      merge_fit<D, U / 2, WITH_V>(p, plain, hq, slice, Sv);
      return;
    }
  }
  merge_body<D, U, WITH_V>(p, plain, hq, slice, Sv);
}

// Workgroup (x, y) of the (B Hq, D / 32) grid takes item xcd_remap(x + y B Hq) in (query head, dim
// slice) order, so a KV head's merges run on the XCD that ran its splits (work_coords' mapping),
// whose L2 still holds the partials just written (config 2's op 26.87 -> 26.52 us).
template <int D, int U, bool WITH_V>
__global__ void __launch_bounds__(256) combine_kernel(const AttnP p, int plain) {
  const int nsl = gridDim.y;
  const int m = xcd_remap(blockIdx.x + blockIdx.y * gridDim.x, gridDim.x * nsl);
  const int64_t hq = m / nsl;
  merge_fit<D, U, WITH_V>(p, plain, hq, m % nsl, merge_count(p, hq));
}

// merge_body with U chosen at run time from the head's partial count.
template <int D>
__device__ void merge_body_rt(const AttnP& p, int64_t hq, int slice) {
  merge_fit<D, MAX_SPLITS / 8, true>(p, 0, hq, slice, merge_count(p, hq));
}

template <int D, bool WITH_V>
inline void launch_combine_u(const AttnP& p, dim3 grid, int plain, hipStream_t s) {
  const int u = (p.num_splits + 7) / 8;
  if (u <= 1) hipLaunchKernelGGL((combine_kernel<D, 1, WITH_V>), grid, dim3(256), 0, s, p, plain);
  else if (u <= 2) hipLaunchKernelGGL((combine_kernel<D, 2, WITH_V>), grid, dim3(256), 0, s, p, plain);
  else if (u <= 4) hipLaunchKernelGGL((combine_kernel<D, 4, WITH_V>), grid, dim3(256), 0, s, p, plain);
  else if (u <= 8) hipLaunchKernelGGL((combine_kernel<D, 8, WITH_V>), grid, dim3(256), 0, s, p, plain);
  else if (u <= 16) hipLaunchKernelGGL((combine_kernel<D, 16, WITH_V>), grid, dim3(256), 0, s, p, plain);
  else hipLaunchKernelGGL((combine_kernel<D, MAX_SPLITS / 8, WITH_V>), grid, dim3(256), 0, s, p, plain);
}

inline hipError_t launch_combine(const AttnP& p, int D, bool plain, hipStream_t s) {
  const bool with_v = p.out != nullptr;
  const dim3 grid(p.B * p.Hq, with_v ? D / 32 : 1);
  const int pl = plain ? 1 : 0;
  if (D == 128) {
    if (with_v) launch_combine_u<128, true>(p, grid, pl, s);
    else launch_combine_u<128, false>(p, grid, pl, s);
  } else {
    if (with_v) launch_combine_u<64, true>(p, grid, pl, s);
    else launch_combine_u<64, false>(p, grid, pl, s);
  }
  return hipGetLastError();
}

// Ragged: S + B chunk slots per KV head (a head has at most that many chunks).
inline dim3 attn_grid(const AttnP& p) {
  return dim3(p.seq_lens != nullptr ? (p.num_splits + p.B) * p.Hkv : p.num_splits * p.Hkv * p.B);
}

// Instantiated group sizes.
#define KVS_FOR_G(X, D) \
  X(D, 1)               \
  X(D, 2)               \
  X(D, 4)               \
  X(D, 7)               \
  X(D, 8)

}  // namespace
}  // namespace kvs
