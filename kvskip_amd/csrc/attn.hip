// Split-K flash-decode kernels for gfx950: dense, block-list (masked), per-block statistics,
// stats-only, fp16 P, single-pass V-skip, two-pass V-skip pass 2, split merges, read ceiling.
//
// Work decomposition. Grid (num_splits, Hkv, B); a workgroup of 4 wavefronts owns one
// contiguous range of "items" (64-token blocks, or entries of a block list) of one KV head
// and serves all G query heads of that head, so each K/V byte is read once. Inside the
// workgroup the 4 wavefronts are independent streams: wavefront w takes items w, w+4, ...
// and keeps its own online-softmax state for the G heads, so the main loop has no
// workgroup barrier. A wavefront processes a whole 64-token block at a time, so the
// per-block statistics fall out of its own registers. The 4 states are merged once, in LDS,
// at the end; with num_splits > 1 the merged state goes to the split partial buffers and a
// second kernel merges the splits.
//
// Lane layouts (64 lanes, D = 64 or 128):
//   K   8 lanes per token row, 8 rows per load; lane (r8 = lane/8, sub = lane%8) holds rows
//       8*rg + r8 (rg = 0..7), dims [8 sub, 8 sub + 8) (+64 for D = 128), as packed bf16.
//       QK = v_dot2_f32_bf16 against the unscaled bf16 query (exact products, fp32 sums),
//       then a 3-step DPP sum over the 8 lanes of the row; the score is scaled after.
//   V   D/8 lanes per row, 8 dims per lane, 16-byte loads; lane accumulates its rows for
//       all G heads in fp32 (acc[G][8]); P reaches the V layout through a per-wavefront
//       LDS tile [64][G] written after the softmax.
// Softmax runs in log2 units (v_exp_f32); per head and block: block max mt, e = 2^(s - mt)
// (the block statistics), p = e * 2^(mt - m_run). K/V rows past T load the last valid row
// and are masked to score -inf.
#include "common.hpp"
#include "internal.hpp"

namespace kvs {
namespace {

constexpr int NWAVE = 4;
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

// Byte range of one (b, head) of a K or V view: rows 0..T-1 of D bf16 each, row stride st.
__device__ __forceinline__ uint32_t head_bytes(int T, int64_t st, int D) {
  return static_cast<uint32_t>((static_cast<int64_t>(T - 1) * st + D) * 2);
}

// K block at token t0: lane (r8, sub) gets rows t0 + 8 rg + r8, 16-byte chunks sub (+8).
// koff = r8 * k_st * 2 + 16 * sub (per lane, fixed); rows past T read as zeros.
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

// Scores of one block in log2 units: s[rg][g] for row 8*rg + lane/8, -inf past T.
template <int D, int G>
__device__ __forceinline__ void qk_block(float (&s)[8][G], const u32x4 (&kr)[8][Lay<D>::KC],
                                         const u32x4 (&qv)[G][Lay<D>::KC], float scale_log2, int t0, int T,
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
    const bool ok = t0 + 8 * rg + r8 < T;
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

// Workgroup epilogue: merge the 4 wavefront states (m, l in log2 units, acc un-normalised),
// then write out/out_f32/lse (one split) or the split partials.
template <int D, int G, bool LOAD_V>
__device__ __forceinline__ void merge_and_store(const AttnP& p, float (&m)[G], float (&l)[G], float (&acc)[G][8],
                                                int b, int h, int split, float* sAcc, float* sMl, bool plain_sum) {
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE;
  constexpr int VLPR = Lay<D>::VLPR;
  if constexpr (LOAD_V) {
    reduce_acc_rows<D, G>(acc);
    if (lane < VLPR) {
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) sAcc[(wave * G + g) * D + 8 * lane + e] = acc[g][e];
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      sMl[(wave * G + g) * 2] = m[g];
      sMl[(wave * G + g) * 2 + 1] = l[g];
    }
  }
  __syncthreads();
  const int S = p.num_splits;
  const int64_t hq0 = static_cast<int64_t>(b) * p.Hq + static_cast<int64_t>(h) * G;
  if constexpr (LOAD_V) {
    for (int o = tid; o < G * D; o += NT) {
      const int g = o / D, d = o % D;
      float A = 0.f, L = 0.f;
      if (plain_sum) {
#pragma unroll
        for (int w = 0; w < NWAVE; ++w) A += sAcc[(w * G + g) * D + d];
        L = 1.f;
      } else {
        float M = NEG_INF;
#pragma unroll
        for (int w = 0; w < NWAVE; ++w) M = fmaxf(M, sMl[(w * G + g) * 2]);
        const float mu = M == NEG_INF ? 0.f : M;
#pragma unroll
        for (int w = 0; w < NWAVE; ++w) {
          const float f = fexp2(sMl[(w * G + g) * 2] - mu);
          L += sMl[(w * G + g) * 2 + 1] * f;
          A += sAcc[(w * G + g) * D + d] * f;
        }
      }
      const int64_t hq = hq0 + g;
      if (S == 1) {
        const float o_ = L > 0.f ? A / L : 0.f;
        p.out[hq * D + d] = f2bf(o_);
        if (p.out_f32) p.out_f32[hq * D + d] = o_;
      } else {
        p.part_acc[(hq * S + split) * D + d] = A;
      }
    }
  }
  if (!plain_sum && tid < G) {
    const int g = tid;
    float M = NEG_INF, L = 0.f;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) M = fmaxf(M, sMl[(w * G + g) * 2]);
    const float mu = M == NEG_INF ? 0.f : M;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) L += sMl[(w * G + g) * 2 + 1] * fexp2(sMl[(w * G + g) * 2] - mu);
    const int64_t hq = hq0 + g;
    if (S == 1) {
      if (p.lse) p.lse[hq] = L > 0.f ? (M + flog2(L)) * LN2 : NEG_INF;
    } else {
      p.part_ml[(hq * S + split) * 2] = M;
      p.part_ml[(hq * S + split) * 2 + 1] = L;
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

// One block's softmax step for head g: updates (m, l), returns the factor c with
// p = e * c, and leaves e = 2^(s - mt) in e[] and the block stats in (mt, st).
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

template <int D, int G, bool MASKED, bool STATS, bool LOAD_V>
__global__ void __launch_bounds__(NT, 2) decode_kernel(const AttnP p) {
  constexpr int GP = gpad<G>();
  __shared__ __attribute__((aligned(16))) float sP[NWAVE][BLK * GP];
  __shared__ __attribute__((aligned(16))) float sAcc[LOAD_V ? NWAVE * G * D : 1];
  __shared__ float sMl[NWAVE * G * 2];

  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE;
  const int r8 = lane >> 3, sub = lane & 7;

  int n_items;
  const int* list = nullptr;
  if constexpr (MASKED) {
    n_items = min(max(p.block_cnt[b * p.Hkv + h], 0), p.max_blocks);
    list = p.block_idx + static_cast<int64_t>(b * p.Hkv + h) * p.max_blocks;
  } else {
    n_items = p.nb;
  }
  const int per = (n_items + p.num_splits - 1) / p.num_splits;
  const int i0 = min(n_items, split * per);
  const int n = min(n_items, i0 + per) - i0;

  const rsrc_t rk = make_rsrc(p.k + b * p.k_sb + h * p.k_sh, head_bytes(p.T, p.k_st, D));
  const rsrc_t rv = make_rsrc(p.v + b * p.v_sb + h * p.v_sh, LOAD_V ? head_bytes(p.T, p.v_st, D) : 0);
  const uint32_t koff = static_cast<uint32_t>(r8 * p.k_st * 2 + 16 * sub);
  const uint32_t voff = static_cast<uint32_t>((lane / Lay<D>::VLPR) * p.v_st * 2 + 16 * (lane % Lay<D>::VLPR));

  u32x4 qv[G][Lay<D>::KC];
  load_q<D, G>(qv, p, b, h, lane);

  float m[G], l[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = NEG_INF;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
  }

  auto block_of = [&](int j) -> int {
    if (j >= n) return -1;
    const int blk = MASKED ? list[i0 + j] : i0 + j;
    return (blk >= 0 && blk < p.nb) ? blk : -1;  // out-of-range list entries are skipped
  };

  u32x4 kr[8][Lay<D>::KC];
  u32x4 vr[Lay<D>::VN];
  float* sPw = sP[wave];

  // Per wavefront: K(j) in flight at the top of iteration j; after QK(j) the V loads of block j
  // and the K loads of the next block are issued together, then PV(j) waits for V(j) only.
  int j = wave;
  int blk = block_of(j);
  if (blk >= 0) load_k_block<D>(kr, rk, koff, p.k_st, blk * BLK);
  for (; j < n; j += NWAVE) {
    const int blk_n = block_of(j + NWAVE);
    float alpha[G];
    if (blk >= 0) {
      const int t0 = blk * BLK;
      float s[8][G];
      qk_block<D, G>(s, kr, qv, p.scale_log2, t0, p.T, lane);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float e[8], mt, st, c;
        block_softmax<G>(s, g, m[g], l[g], e, mt, st, alpha[g], c);
        if constexpr (STATS) {
          const int64_t hq = static_cast<int64_t>(b) * p.Hq + static_cast<int64_t>(h) * G + g;
          if (lane == 0) {
            p.blk_max[hq * p.nb + blk] = mt * LN2;
            p.blk_sum[hq * p.nb + blk] = st;
          }
          if (p.p_out != nullptr && sub == g) {
#pragma unroll
            for (int rg = 0; rg < 8; ++rg) p.p_out[hq * p.t_pad + t0 + 8 * rg + r8] = f2h(e[rg]);
          }
        }
        if constexpr (LOAD_V) {
          if (sub == 0) {
#pragma unroll
            for (int rg = 0; rg < 8; ++rg) sPw[(8 * rg + r8) * GP + g] = e[rg] * c;
          }
        }
      }
      if constexpr (LOAD_V) load_v_block<D>(vr, rv, voff, p.v_st, t0);
    }
    if (blk_n >= 0) load_k_block<D>(kr, rk, koff, p.k_st, blk_n * BLK);
    if constexpr (LOAD_V) {
      if (blk >= 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[g][e] *= alpha[g];
        pv_block<D, G>(acc, vr, sPw, lane);
        __builtin_amdgcn_wave_barrier();
      }
    }
    blk = blk_n;
  }
  merge_and_store<D, G, LOAD_V>(p, m, l, acc, b, h, split, sAcc, sMl, false);
}

// Single-pass V-skip. Per block: QK -> block log-sum-exp per head (log2 units) -> the
// group's vote -> only then the V loads of that block; the next block's K loads are issued
// before the wavefront waits for V, so V(i) overlaps QK(i+1)'s loads.
template <int D, int G>
__global__ void __launch_bounds__(NT, 2) vskip1_kernel(const AttnP p) {
  constexpr int GP = gpad<G>();
  __shared__ __attribute__((aligned(16))) float sP[NWAVE][BLK * GP];
  __shared__ __attribute__((aligned(16))) float sAcc[NWAVE * G * D];
  __shared__ float sMl[NWAVE * G * 2];
  __shared__ float sLse0[G];
  __shared__ int sLoaded[NWAVE];

  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE;
  const int r8 = lane >> 3, sub = lane & 7;
  const int nb = p.nb;
  const int per = (nb + p.num_splits - 1) / p.num_splits;
  const int i0 = min(nb, split * per);
  const int n = min(nb, i0 + per) - i0;
  const rsrc_t rk = make_rsrc(p.k + b * p.k_sb + h * p.k_sh, head_bytes(p.T, p.k_st, D));
  const rsrc_t rv = make_rsrc(p.v + b * p.v_sb + h * p.v_sh, head_bytes(p.T, p.v_st, D));
  const uint32_t koff = static_cast<uint32_t>(r8 * p.k_st * 2 + 16 * sub);
  const uint32_t voff = static_cast<uint32_t>((lane / Lay<D>::VLPR) * p.v_st * 2 + 16 * (lane % Lay<D>::VLPR));
  const int64_t hq0 = static_cast<int64_t>(b) * p.Hq + static_cast<int64_t>(h) * G;

  u32x4 qv[G][Lay<D>::KC];
  load_q<D, G>(qv, p, b, h, lane);
  u32x4 kr[8][Lay<D>::KC];
  u32x4 vr[Lay<D>::VN];

  // Normaliser estimate per head (log2 units): lse_prev, or the block-0 log-sum-exp.
  if (p.lse_prev != nullptr) {
    if (tid < G) sLse0[tid] = p.lse_prev[hq0 + tid] * LOG2E;
  } else if (wave == 0) {
    load_k_block<D>(kr, rk, koff, p.k_st, 0);
    float s[8][G];
    qk_block<D, G>(s, kr, qv, p.scale_log2, 0, p.T, lane);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float x = s[0][g];
#pragma unroll
      for (int rg = 1; rg < 8; ++rg) x = fmaxf(x, s[rg][g]);
      const float mt = max_rows8(x);
      float sum = 0.f;
#pragma unroll
      for (int rg = 0; rg < 8; ++rg) sum += fexp2(s[rg][g] - mt);
      const float lse0 = mt + flog2(sum_rows8(sum));
      if (lane == 0) sLse0[g] = lse0;
    }
  }
  __syncthreads();
  float lse0[G];
#pragma unroll
  for (int g = 0; g < G; ++g) lse0[g] = sLse0[g];

  float m[G], l[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = NEG_INF;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
  }
  float* sPw = sP[wave];
  int loaded = 0;

  int j = wave;
  if (j < n) load_k_block<D>(kr, rk, koff, p.k_st, (i0 + j) * BLK);
  for (; j < n; j += NWAVE) {
    const int blk = i0 + j;
    const int t0 = blk * BLK;
    float s[8][G];
    qk_block<D, G>(s, kr, qv, p.scale_log2, t0, p.T, lane);
    // Per head: block stats and the vote; the softmax update and P are computed as if the block
    // were kept and committed only if the group keeps it.
    float tm[G], tl[G], ta[G];
    bool need = blk == 0 || blk >= nb - p.local;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float x = s[0][g];
#pragma unroll
      for (int rg = 1; rg < 8; ++rg) x = fmaxf(x, s[rg][g]);
      const float mt = max_rows8(x);
      const float mtu = mt == NEG_INF ? 0.f : mt;
      float e[8], sum = 0.f;
#pragma unroll
      for (int rg = 0; rg < 8; ++rg) {
        e[rg] = fexp2(s[rg][g] - mtu);
        sum += e[rg];
      }
      const float st = sum_rows8(sum);
      need = need || (mtu + flog2(st) - lse0[g] >= p.log2_tau);
      const float m_new = fmaxf(m[g], mt);
      const float mu = m_new == NEG_INF ? 0.f : m_new;
      ta[g] = fexp2(m[g] - mu);
      const float c = mt == NEG_INF ? 0.f : fexp2(mt - mu);
      tl[g] = l[g] * ta[g] + st * c;
      tm[g] = m_new;
      if (sub == 0) {
#pragma unroll
        for (int rg = 0; rg < 8; ++rg) sPw[(8 * rg + r8) * GP + g] = e[rg] * c;
      }
    }
    if (need) {
      ++loaded;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        m[g] = tm[g];
        l[g] = tl[g];
#pragma unroll
        for (int u = 0; u < 8; ++u) acc[g][u] *= ta[g];
      }
      load_v_block<D>(vr, rv, voff, p.v_st, t0);
    }
    if (j + NWAVE < n) load_k_block<D>(kr, rk, koff, p.k_st, (blk + NWAVE) * BLK);
    if (need) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      pv_block<D, G>(acc, vr, sPw, lane);
      __builtin_amdgcn_wave_barrier();
    }
  }
  if (lane == 0) sLoaded[wave] = loaded;
  merge_and_store<D, G, true>(p, m, l, acc, b, h, split, sAcc, sMl, false);
  if (tid == 0 && p.vcount != nullptr) {
    int tot = 0;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) tot += sLoaded[w];
    atomicAdd(p.vcount + b * p.Hkv + h, tot);
  }
}

// Two-pass V-skip, pass 2: acc = sum over listed blocks of (blk_scale * P) . V; the weights
// are normalised already, so no softmax and the splits simply add up.
template <int D, int G>
__global__ void __launch_bounds__(NT, 2) pv_kernel(const AttnP p) {
  constexpr int GP = gpad<G>();
  __shared__ __attribute__((aligned(16))) float sP[NWAVE][BLK * GP];
  __shared__ __attribute__((aligned(16))) float sAcc[NWAVE * G * D];
  __shared__ float sMl[NWAVE * G * 2];

  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE;
  const int n_items = min(max(p.block_cnt[b * p.Hkv + h], 0), p.max_blocks);
  const int* list = p.block_idx + static_cast<int64_t>(b * p.Hkv + h) * p.max_blocks;
  const int per = (n_items + p.num_splits - 1) / p.num_splits;
  const int i0 = min(n_items, split * per);
  const int n = min(n_items, i0 + per) - i0;
  const rsrc_t rv = make_rsrc(p.v + b * p.v_sb + h * p.v_sh, head_bytes(p.T, p.v_st, D));
  const uint32_t voff = static_cast<uint32_t>((lane / Lay<D>::VLPR) * p.v_st * 2 + 16 * (lane % Lay<D>::VLPR));
  const int64_t hq0 = static_cast<int64_t>(b) * p.Hq + static_cast<int64_t>(h) * G;

  float m[G], l[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = 0.f;
    l[g] = 1.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
  }
  u32x4 vr[Lay<D>::VN];
  float* sPw = sP[wave];
  const int pg = lane >> 3, ppart = lane & 7;  // P staging: head pg, tokens 8*ppart .. +8
  for (int j = wave; j < n; j += NWAVE) {
    const int blk = list[i0 + j];
    if (blk < 0 || blk >= p.nb) continue;
    const int t0 = blk * BLK;
    load_v_block<D>(vr, rv, voff, p.v_st, t0);
    if (pg < G) {
      const float f = p.blk_scale[((static_cast<int64_t>(b) * p.Hkv + h) * p.nb + blk) * G + pg];
      const u32x4 raw = ld16(p.p_in + (hq0 + pg) * p.t_pad + t0 + 8 * ppart);
      const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        sPw[(8 * ppart + 2 * u) * GP + pg] = h2f(static_cast<uint16_t>(w[u] & 0xffffu)) * f;
        sPw[(8 * ppart + 2 * u + 1) * GP + pg] = h2f(static_cast<uint16_t>(w[u] >> 16)) * f;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    pv_block<D, G>(acc, vr, sPw, lane);
    __builtin_amdgcn_wave_barrier();
  }
  merge_and_store<D, G, true>(p, m, l, acc, b, h, split, sAcc, sMl, true);
}

// Log-sum-exp merge of the split partials; one workgroup per (b, query head), one thread
// per dim. With out == nullptr (stats-only) only lse is produced.
template <int D>
__global__ void __launch_bounds__(D) combine_kernel(const AttnP p) {
  const int64_t hq = blockIdx.x;
  const int d = threadIdx.x;
  const int S = p.num_splits;
  const float* ml = p.part_ml + hq * S * 2;
  float M = NEG_INF;
  for (int s = 0; s < S; ++s) M = fmaxf(M, ml[2 * s]);
  const float mu = M == NEG_INF ? 0.f : M;
  float L = 0.f, A = 0.f;
  const bool with_v = p.out != nullptr;
  for (int s = 0; s < S; ++s) {
    const float w = fexp2(ml[2 * s] - mu);
    L += ml[2 * s + 1] * w;
    if (with_v) A += p.part_acc[(hq * S + s) * D + d] * w;
  }
  if (with_v) {
    const float o = L > 0.f ? A / L : 0.f;
    p.out[hq * D + d] = f2bf(o);
    if (p.out_f32) p.out_f32[hq * D + d] = o;
  }
  if (d == 0 && p.lse) p.lse[hq] = L > 0.f ? (M + flog2(L)) * LN2 : NEG_INF;
}

template <int D>
__global__ void __launch_bounds__(D) combine_sum_kernel(const AttnP p) {
  const int64_t hq = blockIdx.x;
  const int d = threadIdx.x;
  float A = 0.f;
  for (int s = 0; s < p.num_splits; ++s) A += p.part_acc[(hq * p.num_splits + s) * D + d];
  p.out[hq * D + d] = f2bf(A);
  if (p.out_f32) p.out_f32[hq * D + d] = A;
}

// Streaming read of n 16-byte words, grid-stride, XOR-folded so the loads stay live.
__global__ void __launch_bounds__(256) read_kernel(const u32x4* __restrict__ x, int64_t n, uint32_t* out) {
  uint32_t a = 0;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  for (; i + 3 * stride < n; i += 4 * stride) {
    const u32x4 v0 = ld16_nt(x + i), v1 = ld16_nt(x + i + stride);
    const u32x4 v2 = ld16_nt(x + i + 2 * stride), v3 = ld16_nt(x + i + 3 * stride);
    a ^= v0.x ^ v0.y ^ v0.z ^ v0.w ^ v1.x ^ v1.y ^ v1.z ^ v1.w;
    a ^= v2.x ^ v2.y ^ v2.z ^ v2.w ^ v3.x ^ v3.y ^ v3.z ^ v3.w;
  }
  for (; i < n; i += stride) {
    const u32x4 v = ld16_nt(x + i);
    a ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (a == 0x9e3779b9u) out[0] = a;
}

template <int D, int G, bool M, bool ST, bool LV>
hipError_t launch_decode_t(const AttnP& p, hipStream_t s) {
  const dim3 grid(p.num_splits, p.Hkv, p.B);
  hipLaunchKernelGGL((decode_kernel<D, G, M, ST, LV>), grid, dim3(NT), 0, s, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (p.num_splits > 1) {
    hipLaunchKernelGGL((combine_kernel<D>), dim3(p.B * p.Hq), dim3(D), 0, s, p);
    e = hipGetLastError();
  }
  return e;
}

template <int D, int G>
hipError_t dispatch_flags(const AttnP& p, bool masked, bool stats, bool load_v, hipStream_t s) {
  if (!masked && !stats && load_v) return launch_decode_t<D, G, false, false, true>(p, s);
  if (!masked && stats && load_v) return launch_decode_t<D, G, false, true, true>(p, s);
  if (!masked && stats && !load_v) return launch_decode_t<D, G, false, true, false>(p, s);
  if (masked && !stats && load_v) return launch_decode_t<D, G, true, false, true>(p, s);
  if (masked && stats && load_v) return launch_decode_t<D, G, true, true, true>(p, s);
  if (masked && stats && !load_v) return launch_decode_t<D, G, true, true, false>(p, s);
  return hipErrorInvalidValue;
}

template <int D, int G>
hipError_t launch_vskip1_t(const AttnP& p, hipStream_t s) {
  const dim3 grid(p.num_splits, p.Hkv, p.B);
  hipLaunchKernelGGL((vskip1_kernel<D, G>), grid, dim3(NT), 0, s, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (p.num_splits > 1) {
    hipLaunchKernelGGL((combine_kernel<D>), dim3(p.B * p.Hq), dim3(D), 0, s, p);
    e = hipGetLastError();
  }
  return e;
}

template <int D, int G>
hipError_t launch_pv_t(const AttnP& p, hipStream_t s) {
  const dim3 grid(p.num_splits, p.Hkv, p.B);
  hipLaunchKernelGGL((pv_kernel<D, G>), grid, dim3(NT), 0, s, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (p.num_splits > 1) {
    hipLaunchKernelGGL((combine_sum_kernel<D>), dim3(p.B * p.Hq), dim3(D), 0, s, p);
    e = hipGetLastError();
  }
  return e;
}

// Instantiated group sizes.
#define KVS_FOR_G(X, D) \
  X(D, 1)               \
  X(D, 2)               \
  X(D, 4)               \
  X(D, 7)               \
  X(D, 8)

}  // namespace

bool attn_supported(int D, int G) {
  return (D == 64 || D == 128) && (G == 1 || G == 2 || G == 4 || G == 7 || G == 8);
}

hipError_t launch_decode(const AttnP& p, int D, int G, bool masked, bool stats, bool load_v, hipStream_t s) {
#define KVS_CASE(DD, GG) \
  if (D == DD && G == GG) return dispatch_flags<DD, GG>(p, masked, stats, load_v, s);
  KVS_FOR_G(KVS_CASE, 64)
  KVS_FOR_G(KVS_CASE, 128)
#undef KVS_CASE
  return hipErrorInvalidValue;
}

hipError_t launch_vskip1(const AttnP& p, int D, int G, hipStream_t s) {
#define KVS_CASE(DD, GG) \
  if (D == DD && G == GG) return launch_vskip1_t<DD, GG>(p, s);
  KVS_FOR_G(KVS_CASE, 64)
  KVS_FOR_G(KVS_CASE, 128)
#undef KVS_CASE
  return hipErrorInvalidValue;
}

hipError_t launch_pv(const AttnP& p, int D, int G, hipStream_t s) {
#define KVS_CASE(DD, GG) \
  if (D == DD && G == GG) return launch_pv_t<DD, GG>(p, s);
  KVS_FOR_G(KVS_CASE, 64)
  KVS_FOR_G(KVS_CASE, 128)
#undef KVS_CASE
  return hipErrorInvalidValue;
}

hipError_t launch_read(const void* x, int64_t bytes, uint32_t* out, int blocks, hipStream_t s) {
  hipLaunchKernelGGL(read_kernel, dim3(blocks), dim3(256), 0, s, reinterpret_cast<const u32x4*>(x), bytes / 16,
                     out);
  return hipGetLastError();
}

}  // namespace kvs
