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

// Row t of KV head h of sequence b: in a view (k + b k_sb + h k_sh + t k_st) or, with a block table
// (paged cache, k_sb the page stride), row t % 64 of page tbl[b bt + t / 64]; null for a page id
// outside [0, npages).
__device__ __forceinline__ const uint16_t* key_row(const uint16_t* k, int64_t k_sb, int64_t k_sh, int64_t k_st, int b,
                                                   int h, int t, const int32_t* tbl, int64_t bt, int npages) {
  if (tbl == nullptr) return k + b * k_sb + h * k_sh + static_cast<int64_t>(t) * k_st;
  const int pg = tbl[static_cast<int64_t>(b) * bt + t / BLK];
  if (pg < 0 || pg >= npages) return nullptr;
  return k + static_cast<int64_t>(pg) * k_sb + h * k_sh + static_cast<int64_t>(t % BLK) * k_st;
}

__device__ __forceinline__ float clamped_logit(float x) {
  x = fminf(fmaxf(x, 1e-6f), 1.f - 1e-6f);
  return __logf(x) - __logf(1.f - x);
}

// Merge (m, s) log-sum-exp pairs: (m1, s1) <- (m1, s1) + (m2, s2); a pair with s <= 0 is empty.
// Branch-free (selects), so merges of independent pairs interleave.
__device__ __forceinline__ void lse_merge(float& m1, float& s1, float m2, float s2) {
  const bool h1 = s1 > 0.f, h2 = s2 > 0.f;
  const float m = h1 ? (h2 ? fmaxf(m1, m2) : m1) : m2;
  const float a = h1 ? s1 * __expf(m1 - m) : 0.f;
  const float b = h2 ? s2 * __expf(m2 - m) : 0.f;
  s1 = (h1 || h2) ? a + b : s1;
  m1 = (h1 || h2) ? m : m1;
}

// Whole-wavefront log-sum-exp of per-lane (m, s) pairs: max, then rescaled sums (uniform result).
__device__ __forceinline__ void lse_wave(float& m, float& s) {
  const float M = wave_max(s > 0.f ? m : NEG_INF);
  const float S = wave_sum(s > 0.f ? s * __expf(m - M) : 0.f);
  m = M;
  s = S;
}

constexpr int MAX_NB = 4096;   // planner block capacity: update holds a head's blocks in registers

// ---- Two-kernel plan (with a workspace): plan_scores spreads the centroid pass of a head over
// ceil(nb / 32) workgroups (4 wavefronts, 8 block rows each), each publishing per query head the
// (m, s) log-sum-exp of its unattended blocks' estimates and the 32-bit mask of its attended
// blocks; the decision (plan_decide, or the prologue of the masked pass) merges them, decides and
// compacts from the masks. The kernel boundary publishes the partials; in the one-launch plan
// (kvskip_plan_args.ticket) agent-scope stores and a per-head ticket do, and each head's last
// scores workgroup decides (an agent-scope release per workgroup instead, an L2 write-back each,
// cost more than the launch).
constexpr int WW = 4;                // wavefronts per workgroup
constexpr int WU = 2;                // row groups (4 rows) per wavefront
constexpr int WCB = WW * WU * 4;     // 32 blocks per workgroup
constexpr int WNT = WW * WAVE;
constexpr int DCL = MAX_NB / WCB / WAVE;  // chunks per lane of the decision at capacity

__host__ __device__ constexpr int part_stride(int G) { return 2 * G + 1; }  // m[G], s[G], mask

// Chunks of the scores pass over the capacity T (tokens).
__device__ __forceinline__ int plan_chunks(int T) { return ((T + BLK - 1) / BLK + WCB - 1) / WCB; }

// The plan's decision for NH lists (b, KV head h) = bh[k] = b * Hkv + h from the scores pass's
// partials: one wavefront, uniform results (src/kvskip_attn.py:366-383,
// kernels/kvskip_planner.cu:179-201): per query head the log-sum-exp of the estimates over chunks,
// the missed mass, its calibration, age and flags. Each (list, query head) pair is reduced by a
// team of DLP = 8 lanes: lane t of the team merges chunks t, t + 8, ... in order, then the team
// merges across its lanes (DPP), so the reductions of up to 64 / (8 G) lists run side by side and
// the arithmetic does not depend on how many lists one call takes. mk[k][j] receives the
// attended-block mask of chunk lane + 64 j of list k (0 past the chunks). Every load is issued
// before any is used. With `write` lane 0 stores est and trig, and the advanced age if
// `write_age` (a decision repeated by every workgroup of a pass leaves the age to the update: the
// others still read the old one).
constexpr int DLP = 8;
constexpr int LSI = 8;   // partial slots per team lane of an attended log-sum-exp from partials (<= 64 slots)
static_assert(LSI * DLP == 64, "kvskip_plan_args.lse_slots is validated against 64");

// A scores partial, read (COH) with a relaxed agent-scope atomic load: one that another workgroup
// of the same launch wrote through agent-scope stores, past this XCD's L2 (which may hold a stale
// copy of the line: partials of several workgroups share one).
template <bool COH>
__device__ __forceinline__ float ld_part(const float* a) {
  if constexpr (COH)
    return __uint_as_float(__hip_atomic_load(reinterpret_cast<const uint32_t*>(a), __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT));
  else
    return *a;
}

template <int CTRL>
__device__ __forceinline__ void lse_dpp(float& m, float& s) {
  lse_merge(m, s, dpp<CTRL>(m), dpp<CTRL>(s));
}

template <int G, int NH, bool COH = false>
__device__ __forceinline__ void decide_heads(const kvskip_plan_args& p, const int (&bh)[NH], int lane,
                                             uint32_t (&mk)[NH][DCL], bool (&tr)[NH], bool write,
                                             bool write_age = true) {
  constexpr int SP = part_stride(G);
  constexpr int KW = G * DLP <= WAVE ? WAVE / (G * DLP) : 1;  // lists side by side
  constexpr int CPL = MAX_NB / WCB / DLP;                      // chunks per team lane at capacity
  const int C = plan_chunks(p.T);
  const int pair = lane / DLP, t = lane % DLP;
  const int kr = pair / G, g = pair % G;  // this lane's list (within a round) and query head
  int fl[NH], age0[NH];
  float cal0[NH];
#pragma unroll
  for (int k = 0; k < NH; ++k) {
    const float* pb = p.part + static_cast<int64_t>(bh[k]) * C * SP;
#pragma unroll
    for (int j = 0; j < DCL; ++j) mk[k][j] = __float_as_uint(ld_part<COH>(pb + min(lane + WAVE * j, C - 1) * SP + 2 * G));
  }
  // The per-list values are the same on every lane; read through an index the compiler takes for a
  // per-lane one, they stay in vector registers, where a uniform value would be moved to a scalar
  // register (a wait for its load) before the next loads were issued.
#pragma unroll
  for (int k = 0; k < NH; ++k) {
    int v = bh[k];
    asm volatile("" : "+v"(v));
    age0[k] = p.age[v];
    cal0[k] = (p.calib != nullptr && p.calib_on) ? p.calib[v] : 0.f;
    fl[k] = p.flags[v % p.Hkv];
  }
  float miss[NH];
#pragma unroll
  for (int r = 0; r < NH; r += KW) {
    const int k = min(r + kr, NH - 1);
    int v = bh[k];
    asm volatile("" : "+v"(v));
    const int b = v / p.Hkv, h = v - b * p.Hkv;
    const float* pb = p.part + static_cast<int64_t>(v) * C * SP;
    const int64_t hq = static_cast<int64_t>(b) * p.Hq + static_cast<int64_t>(h) * G + g;
    // the attended log-sum-exp: lse_att, or from the split partials of this step's attended pass
    // (max and sum in log2 units; team lane t takes slots t, t + 8, ...)
    // Every load of the round is issued before any value is used: a load whose value is used in
    // the branch that issues it waits there, one memory round trip per branch.
    float lm[LSI], ls[LSI];
    const bool from_part = p.lse_part != nullptr;
    float2 lx[LSI];
#pragma unroll
    for (int i = 0; i < LSI; ++i) lx[i] = make_float2(NEG_INF, 0.f);
    if (from_part) {  // uniform; slots clamped into [0, lse_slots), the ones past it masked below
#pragma unroll
      for (int i = 0; i < LSI; ++i)
        lx[i] = *reinterpret_cast<const float2*>(p.lse_part + (hq * p.lse_stride + min(t + DLP * i, p.lse_slots - 1)) * 2);
    }
    const float la_mem = from_part ? 0.f : p.lse_att[hq];
    const int NI = (C + DLP - 1) / DLP;  // chunk rounds of the team (uniform)
    float pm[CPL], ps[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {  // clamped into the list's chunks; the ones past C are empty
      pm[i] = NEG_INF;
      ps[i] = 0.f;
      if (i < NI) {
        const int cc = min(t + DLP * i, C - 1);
        pm[i] = ld_part<COH>(pb + cc * SP + g);
        ps[i] = ld_part<COH>(pb + cc * SP + G + g);
      }
    }
#pragma unroll
    for (int i = 0; i < LSI; ++i) {
      const bool in = from_part && t + DLP * i < p.lse_slots;
      lm[i] = in ? lx[i].x * LN2 : NEG_INF;
      ls[i] = in ? lx[i].y : 0.f;
    }
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const bool in = i < NI && t + DLP * i < C;
      pm[i] = in ? pm[i] : NEG_INF;
      ps[i] = in ? ps[i] : 0.f;
    }
    float m = NEG_INF, sv = 0.f;
#pragma unroll
    for (int i = 0; i < CPL; ++i)
      if (i < NI) lse_merge(m, sv, pm[i], ps[i]);
    lse_dpp<DPP_XOR1>(m, sv);
    lse_dpp<DPP_XOR2>(m, sv);
    lse_dpp<DPP_HALF_MIRROR>(m, sv);
    float la = la_mem;
    if (from_part) {
      float am = NEG_INF, as = 0.f;
#pragma unroll
      for (int i = 0; i < LSI; ++i) lse_merge(am, as, lm[i], ls[i]);
      lse_dpp<DPP_XOR1>(am, as);
      lse_dpp<DPP_XOR2>(am, as);
      lse_dpp<DPP_HALF_MIRROR>(am, as);
      la = as > 0.f ? am + __logf(as) : NEG_INF;
    }
    const float e = sv > 0.f ? 1.f / (1.f + __expf(la - (m + __logf(sv)))) : 0.f;
#pragma unroll
    for (int q = 0; q < KW; ++q) {
      if (r + q < NH) {
        float mx = 0.f;
#pragma unroll
        for (int gg = 0; gg < G; ++gg) mx = fmaxf(mx, lane_value(e, DLP * (q * G + gg)));
        miss[r + q] = mx;
      }
    }
  }
#pragma unroll
  for (int k = 0; k < NH; ++k) {
#pragma unroll
    for (int j = 0; j < DCL; ++j)
      if (lane + WAVE * j >= C) mk[k][j] = 0u;
    float dec = miss[k];
    if (p.calib != nullptr && p.calib_on)
      dec = p.calib_kind ? miss[k] + cal0[k] : 1.f / (1.f + __expf(-(clamped_logit(miss[k]) + cal0[k])));
    const int a = age0[k] + 1;
    const bool ix = (fl[k] & 2) != 0;  // a token-index list never refreshes
    tr[k] = !ix && (dec > p.delta || a >= p.max_age || (fl[k] & 1));
    if (write && lane == 0) {
      if (!ix && p.est != nullptr) p.est[bh[k]] = miss[k];
      if (!ix && write_age) p.age[bh[k]] = tr[k] ? 0 : a;
      p.trig[bh[k]] = tr[k] ? 1 : 0;
    }
  }
}

// What the planned pass's decision yields (kvskip_plan_args.decide_mode, KVSKIP_DECIDE_*).
enum DecideMode {
  DECIDE_PLAN = 0,   // plan's decision (trig, est, age) and the list to read: every block or the attended set
  DECIDE_LISTS = 1,  // the attended set's list alone, no decision (trig, est, age untouched)
  DECIDE_POST = 2,   // the decision against a pass's lse_att, and the refresh pass's list: every block
                     // of a refreshing head, none of the others
};

// A decision's lists under a mode (lane holds chunks lane + 64 j of blocks 32 c .. 32 c + 31; nb
// blocks): LISTS refreshes nothing (the attended sets); POST gives a refreshing head the blocks
// outside its attended set (no longer a "read every block" list: tr is cleared) and every other head
// an empty list.
template <int NH>
__device__ __forceinline__ void apply_decide_mode(int mode, uint32_t (&mk)[NH][DCL], bool (&tr)[NH], int lane,
                                                  int nb) {
#pragma unroll
  for (int k = 0; k < NH; ++k) {
#pragma unroll
    for (int j = 0; j < DCL; ++j) {
      const int left = nb - WCB * (lane + WAVE * j);  // blocks of this chunk in the sequence
      const uint32_t valid = left >= WCB ? ~0u : (left > 0 ? (1u << left) - 1u : 0u);
      if (mode == DECIDE_POST) mk[k][j] = tr[k] ? ~mk[k][j] & valid : 0u;
    }
    if (mode != DECIDE_PLAN) tr[k] = false;
  }
}

template <int G, bool COH = false>
__device__ __forceinline__ bool decide_head(const kvskip_plan_args& p, int b, int h, int lane, uint32_t (&mk)[DCL],
                                            bool write, bool write_age = true, int mode = DECIDE_PLAN, int nb = 0) {
  const int bh[1] = {b * p.Hkv + h};
  uint32_t m[1][DCL];
  bool tr[1];
  decide_heads<G, 1, COH>(p, bh, lane, m, tr, write, write_age);
  apply_decide_mode<1>(mode, m, tr, lane, nb);
#pragma unroll
  for (int j = 0; j < DCL; ++j) mk[j] = m[0][j];
  return tr[0];
}

// Exclusive prefix over the wavefront of the attended blocks in the chunks a lane holds (pre[j]
// for chunk lane + 64 j, ascending block order; masks past the C chunks are 0, as the decision
// leaves them); returns the total (uniform). Both chunks' counts go through one scan, packed in the
// two 16-bit halves (a prefix is at most 64 * 32).
__device__ __forceinline__ int mask_prefix(const uint32_t (&mk)[DCL], int lane, int C, int (&pre)[DCL]) {
  static_assert(DCL == 2, "two chunks per lane");
  (void)lane;
  (void)C;
  const int n0 = __popc(mk[0]), n1 = __popc(mk[1]);
  const int incl = wave_incl_scan(n0 | (n1 << 16));
  const int tot = __builtin_amdgcn_readlane(incl, WAVE - 1);
  const int tot0 = tot & 0xFFFF;
  pre[0] = (incl & 0xFFFF) - n0;
  pre[1] = tot0 + (incl >> 16) - n1;
  return tot0 + (tot >> 16);
}

// List positions [a0 - 1, a1) of the ascending attended blocks, into out[pos - a0 + 1], from the
// chunk masks and their exclusive prefixes in shared memory (mk[c], pre[c] for the C chunks, as
// mask_prefix gives them; chunk c holds blocks 32 c + bit), by a team of `stride` threads (this
// one t): each thread takes blocks t, t + stride, ... and places a marked block at its list
// position if that falls in the range. Position -1 (before the list) is the caller's. No thread
// loops over set bits, so a slice costs about C * 32 / stride steps of a few instructions. Signed
// arithmetic throughout (with an unsigned rank, a0 = 0 would make a0 - 1 the largest value).
__host__ __device__ __forceinline__ void slice_from_masks(const uint32_t* mk, const int* pre, int C, int a0, int a1,
                                                          int* out, int t, int stride) {
  for (int i = t; i < C * WCB; i += stride) {
    const uint32_t m = mk[i / WCB];
    const int bit = i % WCB;
    if ((m >> bit) & 1u) {
      const int r = pre[i / WCB] + static_cast<int>(__builtin_popcount(m & ((1u << bit) - 1u)));
      if (r >= a0 - 1 && r < a1) out[r - a0 + 1] = i;
    }
  }
}

// The head's block list and count from its decision: every block (refresh) or the ascending
// attended blocks of the chunk masks. One wavefront.
__device__ __forceinline__ void write_block_list(const kvskip_plan_args& p, int64_t bh, int nb, bool tr,
                                                 const uint32_t (&mk)[DCL], int lane) {
  int* bi = p.block_idx + bh * p.NBC;
  if (tr) {  // refresh: every block
    for (int i = lane; i < nb; i += WAVE) bi[i] = i;
    if (lane == 0) p.block_cnt[bh] = nb;
    return;
  }
  int pre[DCL];
  const int cnt = mask_prefix(mk, lane, plan_chunks(p.T), pre);
#pragma unroll
  for (int j = 0; j < DCL; ++j) {
    int off = pre[j];
    for (uint32_t m = mk[j]; m != 0; m &= m - 1) bi[off++] = (lane + WAVE * j) * WCB + __ffs(m) - 1;
  }
  if (lane == 0) p.block_cnt[bh] = cnt;
}

// An update carried by a pass runs in the pass's NWAVE-wavefront workgroups, over up to
// CARRY_MAX_R * 64 blocks (longer: its own launch first). R = 24 (1025..1536 blocks, B 32 at 64k)
// still fits the pass's registers; R = 32 did not.
constexpr int carry_waves(int G) { return G < NWAVE ? G : NWAVE; }
constexpr int CARRY_MAX_R = 24;

// Order-preserving key of a float (larger float -> larger key).
__device__ __forceinline__ uint32_t fkey(float y) {
  const uint32_t u = __float_as_uint(y);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Top-p cut of one query head held across a wavefront (lane: blocks lane + 64 r, r < R; slots r >= RU
// hold no block, RU uniform): the largest key theta of y = x - lse whose upper set {key >= theta}
// holds >= level of the mass w = exp(y), i.e. the fewest blocks reaching level with ties at the cut
// kept (kernels/kvskip.py:140-143 keeps the blocks whose heavier blocks hold < level); theta = 0
// (every block) when the whole mass falls short of level. Uniform result. w > 0 exactly where a
// block holds mass; ymax = max y, with w of that block = __expf(ymax).
//
// Radix select over the key less the smallest key of a block with mass (kmin), 8 bits per pass from
// the top bit of the span up to the largest key (that of ymax, the largest y). A pass sums the
// blocks still in play (offset key above the bits decided so far equal to them) into 256 bins of the
// next 8 bits and takes the highest bin whose mass from the top reaches what is still needed; a bin
// holding one block ends the search at that block's key. Bins over the span spread the blocks (few
// LDS atomics to one address). Each bin packs the count of its blocks (bits 51..63) over their mass
// in 2^-48 fixed point (a head's mass, about 1, stays under 2^49, so the fields never carry into each
// other): the sums are exact, the passes agree with each other and the result does not depend on the
// order of the adds. hist: this wavefront's 256 LDS bins, used by it alone.
constexpr int BIN_CNT_SHIFT = 51;
constexpr uint64_t BIN_MASS = (1ull << BIN_CNT_SHIFT) - 1;

__device__ __forceinline__ uint64_t fixmass(float w) {  // floor(w 2^48), w in [0, 8)
  const float s = w * 0x1p16f;                        // exact
  const uint32_t hi = static_cast<uint32_t>(s);
  const float f = s - static_cast<float>(hi);         // exact fraction of s
  return (static_cast<uint64_t>(hi) << 32) | static_cast<uint32_t>(f * 0x1p32f);
}

template <int CTRL>
__device__ __forceinline__ uint64_t dpp64(uint64_t v) {  // 0 where the source lane is out of the row
  const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, true);
  const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(v >> 32), CTRL, 0xF, 0xF, true);
  return (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo);
}

__device__ __forceinline__ uint64_t lane64(uint64_t v, int src) {
  const uint32_t lo = __builtin_amdgcn_readlane(static_cast<int>(v), src);
  const uint32_t hi = __builtin_amdgcn_readlane(static_cast<int>(v >> 32), src);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// Inclusive scan over the lanes (lane 0 first) of a 64-bit sum: DPP shifts inside each 16-lane
// row, then the totals of the rows before.
__device__ __forceinline__ uint64_t wave_scan64(uint64_t v, int lane) {
  v += dpp64<0x111>(v);  // row_shr:1
  v += dpp64<0x112>(v);  // row_shr:2
  v += dpp64<0x114>(v);  // row_shr:4
  v += dpp64<0x118>(v);  // row_shr:8
  const uint64_t t0 = lane64(v, 15), t1 = lane64(v, 31), t2 = lane64(v, 47);
  const int row = lane >> 4;
  return v + (row == 0 ? 0 : row == 1 ? t0 : row == 2 ? t0 + t1 : t0 + t1 + t2);
}

template <int R>
__device__ __forceinline__ uint32_t topp_theta(const uint32_t (&key)[R], const float (&w)[R], int RU, float level,
                                               float ymax, uint64_t* hist) {
  const int lane = threadIdx.x % WAVE;
  uint64_t need = fixmass(level);  // mass still needed from the blocks in play
  if (fixmass(__expf(ymax)) >= need) return fkey(ymax);  // the heaviest block alone reaches level
  // Blocks lighter than wcut are out of play: together they hold < (1 - level) / 8, so the blocks
  // above them hold >= level and the cut lies among those (with room for the rounding of w; none
  // are left out for level within 1e-5 of 1).
  const float wcut = level < 0.99999f ? (1.f - level) / (8.f * WAVE * RU) : 0.f;
  uint64_t inc = 0;  // bit r: slot r in play
  uint32_t kmin = ~0u;
#pragma unroll
  for (int r = 0; r < R; ++r)
    if (r < RU && w[r] > wcut) {
      inc |= 1ull << r;
      kmin = min(kmin, key[r]);
    }
  kmin = wave_min_u32(kmin);
  const uint32_t kmax = fkey(ymax);
  if (kmax < kmin) return 0;  // no block holds mass
  const uint32_t span = kmax - kmin;
  int sh = span == 0 ? 0 : max(24 - static_cast<int>(__builtin_clz(span)), 0);  // top 8 bits of the span
  int prev = 32;              // offset bits >= prev are decided (none yet)
  uint32_t dec = 0;           // the decided offset bits
  uint64_t* mine = hist + 4 * (WAVE - 1 - lane);  // lane L holds bins 4 (63 - L) .. + 3: lane 0 the top
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {  // the span has <= 32 bits: <= 4 passes
#pragma unroll
    for (int k = 0; k < 4; ++k) mine[k] = 0;
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t off = key[r] - kmin;
      if (((inc >> r) & 1) && (pass == 0 || (off >> prev) == (dec >> prev)))
        __hip_atomic_fetch_add(hist + ((off >> sh) & 255u), (1ull << BIN_CNT_SHIFT) | fixmass(w[r]),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    uint64_t h[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) h[k] = mine[k];
    const uint64_t s3 = h[3], s2 = h[2] + s3, s1 = h[1] + s2, s0 = h[0] + s1;  // from bin k up, in the lane
    const uint64_t incl = wave_scan64(s0, lane);  // bins >= 4 (63 - lane)
    const uint64_t excl = incl - s0;
    const uint64_t reach = __ballot((incl & BIN_MASS) >= need);
    if (reach == 0) return 0;                      // only in the first pass: the whole mass < level
    const int L = __builtin_ctzll(reach);          // the lane of the highest bin that reaches need
    const int k = ((excl + s3) & BIN_MASS) >= need ? 3 : ((excl + s2) & BIN_MASS) >= need ? 2
                : ((excl + s1) & BIN_MASS) >= need ? 1 : 0;
    const uint64_t hk = k == 3 ? s3 : k == 2 ? s2 - s3 : k == 1 ? s1 - s2 : s0 - s1;
    const uint64_t above = excl + (k == 3 ? s3 : k == 2 ? s2 : k == 1 ? s1 : s0) - hk;  // bins over the chosen
    const uint32_t bin = 4 * (WAVE - 1 - L) + __builtin_amdgcn_readlane(k, L);
    const uint64_t hb = lane64(hk, L);
    need -= lane64(above, L) & BIN_MASS;
    dec |= bin << sh;
    if (sh == 0) break;
    if ((hb >> BIN_CNT_SHIFT) == 1) {  // one block in the bin: the cut is its key
      uint32_t mk = 0;
      bool has = false;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint32_t off = key[r] - kmin;
        const bool c = ((inc >> r) & 1) && (pass == 0 || (off >> prev) == (dec >> prev)) && ((off >> sh) & 255u) == bin;
        mk = c ? key[r] : mk;
        has = has || c;
      }
      return __builtin_amdgcn_readlane(mk, __builtin_ctzll(__ballot(has)));
    }
    prev = sh;
    sh = max(sh - 8, 0);
  }
  return kmin + dec;
}

// Update of (b, KV head h): src/kvskip_attn.py:386-391 (_calib_learn 302-320, _refresh_state
// 182-199, _attended_lse 282-288) on the device, as kernels/kvskip_planner.cu:229-305.
// Wavefront w < NWV takes query heads g = w + NWV j of the group (HPW = ceil(G / NWV) per
// wavefront); lane holds blocks i = lane + 64 r, r < R (nb <= 64 R). Wavefronts >= NWV of a wider
// workgroup only pass the barrier.
template <int G, int R, int NWV>
__device__ __forceinline__ void update_body(const kvskip_update_args& p, int h, int b) {
  constexpr int HPW = (G + NWV - 1) / NWV;
  constexpr int RC = R <= 16 ? R : (R % 16 == 0 ? 16 : 8);  // register slots whose loads are in flight together
  if (threadIdx.x >= NWV * WAVE) {
    __syncthreads();
    return;
  }
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE;
  const int nbl = (p.T + BLK - 1) / BLK;                       // row length of the statistics
  const int64_t bh = static_cast<int64_t>(b) * p.Hkv + h;
  const int64_t hrow0 = static_cast<int64_t>(b) * p.Hq + static_cast<int64_t>(h) * G;  // head g: hrow0 + g
  __shared__ uint64_t sKm[G][R];  // each query head's top-p blocks (lane bits of r)
  __shared__ float sReal[G];
  __shared__ uint64_t sHist[NWV][256];  // each wavefront's top-p histogram
  uint8_t* keep = p.keep + bh * p.NBC;
  const uint8_t* ixp = p.idx != nullptr ? p.idx + static_cast<int64_t>(b) * p.NBC : keep;  // keep: stand-in
  // The sequence's length and the head's flags, trigger, latch and calibration are read through
  // indices the compiler takes for per-lane ones, without branches: as uniform values they went to
  // scalar registers, a wait for each load before the statistics loads below were issued. Where a
  // pointer may be null, the block statistics stand in (read only here, at least B Hkv entries;
  // the value is then unused).
  int bv = b, hv = h, bhv = static_cast<int>(bh);
  asm volatile("" : "+v"(bv), "+v"(hv), "+v"(bhv));
  const float* sti = p.blk_max;
  const int32_t sl = (p.seq_lens != nullptr ? p.seq_lens : reinterpret_cast<const int32_t*>(sti))[bv];
  const bool tr = p.trig[bhv] != 0;
  const int fl_raw = (p.flags != nullptr ? p.flags : reinterpret_cast<const int32_t*>(sti))[hv];
  const uint8_t ax_raw = (p.aix != nullptr ? p.aix : reinterpret_cast<const uint8_t*>(sti))[bhv];
  const float est_raw = (p.calib != nullptr ? p.est : sti)[bhv];
  const float cal_raw = (p.calib != nullptr ? p.calib : sti)[bhv];
  const int fl = p.flags != nullptr ? fl_raw : 0;
  const bool uni = (p.idx != nullptr) & (((fl & 4) != 0) | ((p.aix != nullptr) & (ax_raw != 0)));
  const bool ixh = (fl & 2) != 0;  // token-index head: read index + sink + local (list_stats)
  const float est0 = p.calib != nullptr ? est_raw : 0.f;
  const float cal0 = p.calib != nullptr ? cal_raw : 0.f;

  const int nb = ((p.seq_lens != nullptr ? min(max(sl, 1), p.T) : p.T) + BLK - 1) / BLK;  // the sequence's blocks (seq_T's rule)
  float x[HPW][R];     // block log-weights blk_max + log blk_sum (-inf where not read / past nb)
  uint64_t kp = 0;     // bit r: block in the stored set before this update
  uint64_t att = 0;    // bit r: block attended this step (stored set + sink + local + index union)
#pragma unroll
  for (int c = 0; c < R; c += RC) {
    float bm[HPW][RC], bs[HPW][RC];
    uint32_t kb[RC], ib[RC];
#pragma unroll
    for (int r = 0; r < RC; ++r) {  // loads of the chunk first, clamped into the row (slots past nb masked)
      const int ic = min(lane + WAVE * (c + r), nbl - 1);
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
      // cs_now of the refresh: the first CN slots in flight during the search, the rest loaded in
      // groups of CN below (a group's loads issued before its stores: the stores may alias them, so a
      // load per slot placed after the previous slot's stores waited a round trip each)
      constexpr int CN = R <= 16 ? R : (R % 16 == 0 ? 16 : 8);
      float cn[CN];
#pragma unroll
      for (int r = 0; r < CN; ++r) cn[r] = p.cs_now[hrow * p.NBC + min(lane + WAVE * r, nb - 1)];
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
      const uint32_t theta = topp_theta<R>(key, w, RU, p.level, mx - lse, sHist[wave]);
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
      for (int c0 = 0; c0 < R; c0 += CN) {
        float cc[CN];
        if (c0 == 0 || WAVE * c0 < nb) {  // uniform: a group past the sequence stores only the tail values
#pragma unroll
          for (int r = 0; r < CN; ++r)
            cc[r] = c0 == 0 ? cn[r] : p.cs_now[hrow * p.NBC + min(lane + WAVE * (c0 + r), nb - 1)];
        } else {
#pragma unroll
          for (int r = 0; r < CN; ++r) cc[r] = 0.f;
        }
#pragma unroll
        for (int r = 0; r < CN; ++r) {
          const int i = lane + WAVE * (c0 + r);
          if (i < p.NBC) {
            p.lse_ref[hrow * p.NBC + i] = x[j][c0 + r];
            p.cs_ref[hrow * p.NBC + i] = i < nb ? cc[r] : 0.f;
          }
        }
      }
      for (int i = WAVE * R + lane; i < p.NBC; i += WAVE) {
        p.lse_ref[hrow * p.NBC + i] = NEG_INF;
        p.cs_ref[hrow * p.NBC + i] = 0.f;
      }
    }
  }
  __syncthreads();  // every read of the old stored set is done; sKm / sReal complete

  if (p.age != nullptr && tid == 0 && !(fl & 2)) p.age[bh] = tr ? 0 : p.age[bh] + 1;  // a pass's decision
  if (tr && p.calib != nullptr && tid == 0) {
    float real = 0.f;
    for (int g = 0; g < G; ++g) real = fmaxf(real, sReal[g]);
    const float resid = p.calib_kind ? real - est0 : clamped_logit(real) - clamped_logit(est0);
    float c = p.calib_kind == 2 ? fmaxf((1.f - p.calib_rate) * cal0, resid)
                                : (1.f - p.calib_rate) * cal0 + p.calib_rate * resid;
    if (!p.calib_free) c = fmaxf(c, 0.f);
    p.calib[bh] = c;
    if (p.aix != nullptr && c > p.aix_thr) p.aix[bh] = 1;
  } else if (p.calib != nullptr && p.aix != nullptr && tid == 0 && cal0 > p.aix_thr) {
    // the latch looks at every head's correction, not only the refreshing heads'
    // (src/kvskip_attn.py:318-319): an unchanged correction above a threshold the head never
    // crossed while refreshing (a threshold below the initial 0) latches it too
    p.aix[bh] = 1;
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
