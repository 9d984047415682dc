// Fused grouped-query attention for gfx950 (head_dim 64).
//
// Replaces the reference's per-head chain  score GEMM -> (masked) softmax ->
// P.V GEMM  (vla/text_encoder_bf16.py:502-526, vla/vision_block_bf16.py:325-367,
// vla/action_expert_bf16.py:689-713, 764-787) with one kernel per call.
// Numerics follow the torch modules (vla/text_encoder_bf16.py:117-126):
// scores and the running maximum in fp32, probabilities rounded to bf16 before
// the P.V product, fp32 accumulation, bf16 output.  The softmax denominator is
// the fp32 sum of the same bf16-rounded probabilities that multiply V
// (accumulated on the MFMA), so the normalised weights sum to 1 exactly as
// used; torch sums the unrounded fp32 values, a difference below bf16's
// rounding of the output.
//
// Work decomposition: one workgroup = 64, 128 or 256 query rows of one query
// head (4 waves x 16, 32 or 64 rows); K/V blocks of 64 keys stream through a
// 3-stage LDS ring (see attention_kernel).
#include "svla_common.h"

namespace {

constexpr int D = 64;
constexpr int BKEY = 64;   // keys per LDS stage
// Query rows per wave: QT 16-column MFMA tiles (QT = 2: 32 rows, 128 per
// workgroup; QT = 1 for short query ranges and small grids, QT = 4 for large
// unmasked grids, see the launcher)
template <int QT> constexpr int QW = 16 * QT;
template <int QT> constexpr int BQ = 4 * QW<QT>;
constexpr int kAttnCUs = 256;  // MI355X compute units

struct AttnArgs {
  const bf16* q; long ldq, q_bs;
  const bf16* k; long ldk, k_bs;
  // optional bf16 remainders of fp32 Q and K (same layout and strides as q,
  // k): the scores are then K . Q^T with Q = q + q_lo, K = k + k_lo
  const bf16* q_lo;
  const bf16* k_lo;
  const bf16* v; long ldv, v_bs;
  bf16* o; long ldo, o_bs;
  int sq, sk, hq, hkv;
  float scale_log2;  // scale * log2(e)
  int mask_kind, prefix_len;
};

// Keys a query row may see, as one bound: key j is visible to row i iff
// j < key_limit(i).  causal: j <= i; prefix-LM: j <= i or j < prefix_len
// (the bidirectional prefix block); none: every key.  Always also j < sk.
__device__ __forceinline__ int key_limit(int kind, int qi, int sk, int prefix_len) {
  const int pre = kind == SVLA_MASK_NONE ? sk : (kind == SVLA_MASK_PREFIX_LM ? prefix_len : 0);
  return min(sk, max(qi + 1, pre));
}

// LDS stage = K tile [64 keys][64 d] + V tile [64 keys][64 d], both row-major
// with the 16-byte chunk c of key row r stored in slot c ^ (r & 7), so that
// both the K fragment reads (16 keys x one chunk) and the V transpose reads
// (4 keys x 4 chunks per 16 lanes) spread over the banks.
__device__ __forceinline__ int kv_off(int key, int d) {  // element offset, d % 4 == 0
  return key * D + ((((d >> 3) ^ key) & 7) << 3) + (d & 7);
}

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));

// Maximum of two scores as IEEE 754-2019 maximum (v_maximum3_f32 on gfx950):
// unlike fmaxf (maxNum), which the compiler must precede with a
// canonicalising v_max of each input, it propagates NaN and needs no quieting,
// so a 16-score row maximum is 8 instructions and a shuffle step 1, not 10
// and 3.  For the non-NaN scores here the two agree (masked scores are -inf).
__device__ __forceinline__ float smax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// Reductions over lanes l ^ 16 and l ^ 32 with the gfx950 row-swap VALU ops
// (v_permlane16_swap / v_permlane32_swap): called with both operands = x,
// every lane ends up holding {x[l], x[l ^ 16]} (resp. l ^ 32) in some order.
// No LDS round trip, unlike a ds_bpermute shuffle.
__device__ __forceinline__ float max_xor16(float x) {
  const u32x2_t r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return smax(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
  const u32x2_t r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return smax(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float x) {
  const u32x2_t r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
  const u32x2_t r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
typedef __attribute__((address_space(3))) v4i16* lds_v4i16_ptr;

// V^T operand of O^T += V^T . P^T via the LDS transpose read: within each
// 16-lane group, lane j receives element (j & 3) of the 8-byte chunks of
// lanes (j >> 2) + 4t, t = 0..3.  Lane i = 4t + r of the group points at
// V[kbase + t][dbase + 4r], so lane j gets V[kbase + t][dbase + j], t = 0..3:
// 4 consecutive keys of head dim (dbase + j).
__device__ __forceinline__ v4i16 v_tr_read(const bf16* sv, int kbase, int dbase, int i) {
  const int t = i >> 2, r = i & 3;
  const bf16* p = sv + kv_off(kbase + t, dbase + 4 * r);
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_ptr)(p));
}

// One workgroup = 4 QW query rows of one query head (4 waves x QW rows); the
// loop streams blocks of 64 keys of the head's KV group (h * hkv / hq)
// through a 3-stage ring of LDS buffers filled by global_load_lds.
//
// Products are computed transposed,
//   S^T[key, q] = K . Q^T         (A = K fragment from LDS, B = the wave's Q)
//   O^T[d, q]  += V^T . P^T       (A = V^T via transpose read, B = P^T)
// so that with v_mfma_f32_16x16x32_bf16 each lane owns one query column: the
// online-softmax statistics are lane-local and the row reductions are two
// shuffles (lanes l, l^16, l^32).  The S^T accumulators of two consecutive
// 16-key subtiles are exactly the B operand P^T of the next MFMA (keys
// {4g..4g+3} u {16+4g..16+4g+3} in k-slots 8g..8g+7, g = lane / 16); the V^T
// operand is read with the same key order.
// FULL: no mask and sk % 64 == 0, so no per-score checks at all.
// LO: 0 plain bf16 Q and K; 1 Q = q + q_lo (the fp32 RoPE output as two bf16
// parts: S^T gains K . q_lo^T); 2 also K = k + k_lo (K_lo streams through a
// third ring beside K and V; S^T gains k_lo . q^T).  The reference scores
// the fp32 post-RoPE Q and K (vla/text_encoder_bf16.py:92-104, 117-122).
// With LO > 0 the softmax is also the reference's exactly, in two passes over
// the key blocks: the first takes each query's maximum m and fp32 sum
// l = sum exp(s - m), the second recomputes the scores and rounds
// p = bf16(exp(s - m) * (1 / l)) -- the normalised fp32 probability, as torch's
// softmax(...).to(bf16) -- before P.V (the one-pass form below rounds the
// unnormalised exponentials and divides by the sum of the rounded values at
// the end).  These RoPE'd layers have at most a few hundred keys.
template <bool FULL, int QT, int LO>
__global__ __launch_bounds__(256, 2) void attention_kernel(AttnArgs p) {
  constexpr int QW = ::QW<QT>, BQ = ::BQ<QT>;
  constexpr int KLO = LO == 2 ? BKEY * D : 64;  // K remainder stages (LO == 2 only)
  __shared__ __attribute__((aligned(1024))) bf16 sK0[BKEY * D], sK1[BKEY * D], sK2[BKEY * D];
  __shared__ __attribute__((aligned(1024))) bf16 sV0[BKEY * D], sV1[BKEY * D], sV2[BKEY * D];
  __shared__ __attribute__((aligned(1024))) bf16 sL0[KLO], sL1[KLO], sL2[KLO];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = blockIdx.y, b = blockIdx.z;
  const int kvh = h * p.hkv / p.hq;
  const int q0 = blockIdx.x * BQ;
  const int grp = lane >> 4, col = lane & 15;
  const int qw = q0 + wave * QW;                 // first query row of this wave

  const bf16* qb = p.q + b * p.q_bs + h * D;
  const bf16* kb = p.k + b * p.k_bs + kvh * D;
  const bf16* qlb = LO >= 1 ? p.q_lo + b * p.q_bs + h * D : nullptr;
  const bf16* klb = LO == 2 ? p.k_lo + b * p.k_bs + kvh * D : nullptr;
  const bf16* vb = p.v + b * p.v_bs + kvh * D;

  // last key any row of this workgroup may see
  int kend = p.sk;
  if (!FULL && p.mask_kind != SVLA_MASK_NONE) {
    const int qmax = min(p.sq, q0 + BQ) - 1;
    int lim = qmax + 1;
    if (p.mask_kind == SVLA_MASK_PREFIX_LM) lim = max(lim, p.prefix_len);
    kend = min(kend, lim);
  }
  const int nb = (kend + BKEY - 1) / BKEY;

  // DMA: each stage is 8 + 8 instructions of 1 KB (8 key rows each); wave w
  // issues K and V rows 16w .. 16w+15.  Lane -> key row lane / 8, LDS slot
  // lane % 8 holding logical chunk slot ^ (row & 7).  Rows past sk are
  // clamped (masked or never used).
  long koff[2], voff[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int key = (wave * 2 + j) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ (key & 7);
    koff[j] = (long)key * p.ldk + c * 8;
    voff[j] = (long)key * p.ldv + c * 8;
  }
  auto issue = [&](auto SI, int blk) {
    constexpr int S = decltype(SI)::value;
    bf16* sk = S == 0 ? sK0 : S == 1 ? sK1 : sK2;
    bf16* sv = S == 0 ? sV0 : S == 1 ? sV1 : sV2;
    bf16* sl = S == 0 ? sL0 : S == 1 ? sL1 : sL2;
    blk = min(blk, nb - 1);  // past the end: reload the last block (never read)
    const int k0 = blk * BKEY;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      // block offsets are wave-uniform (scalar); only a partial last block
      // (never in FULL) needs per-lane clamping of rows past sk
      const bf16* gk = kb + (long)k0 * p.ldk + koff[j];
      const bf16* gv = vb + (long)k0 * p.ldv + voff[j];
      long adj = 0;
      if constexpr (!FULL) {
        const int key = (wave * 2 + j) * 8 + (lane >> 3);
        const int rows_left = p.sk - 1 - k0;
        adj = key > rows_left ? (long)(rows_left - key) : 0;
        gk += adj * p.ldk;
        gv += adj * p.ldv;
      }
      __builtin_amdgcn_global_load_lds((void*)gk, (lds_ptr_t)(sk + (wave * 2 + j) * 512), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((void*)gv, (lds_ptr_t)(sv + (wave * 2 + j) * 512), 16, 0, 0);
      if constexpr (LO == 2) {
        const bf16* gl = klb + ((long)k0 + adj) * p.ldk + koff[j];
        __builtin_amdgcn_global_load_lds((void*)gl, (lds_ptr_t)(sl + (wave * 2 + j) * 512), 16, 0, 0);
      }
    }
  };

  // Q fragments (B operand of S^T): rows qw + 16 qt + col, d = 32 ks + 8 grp.
  // Rows past sq are clamped (their outputs are never stored); loading
  // without a branch keeps the loads in flight across the DMA prologue.
  bf16x8 qf[QT][2];
  bf16x8 qlf[LO >= 1 ? QT : 1][2];  // Q remainders (LO >= 1)
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int qi = min(qw + qt * 16 + col, p.sq - 1);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) qf[qt][ks] = ld8(qb + (long)qi * p.ldq + ks * 32 + grp * 8);
    if constexpr (LO >= 1) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) qlf[qt][ks] = ld8(qlb + (long)qi * p.ldq + ks * 32 + grp * 8);
    }
  }

  // o[qt][0..3]: O^T tiles (head dims 16 t .. 16 t + 15); o[qt][4]: the
  // softmax denominator, accumulated by the MFMA with an all-ones V^T operand
  // (every row of that tile holds sum_k bf16(p[q, k]) for the lane's query q),
  // so it is rescaled with the outputs and needs no VALU sums or shuffles
  f32x4 o[QT][5];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
#pragma unroll
    for (int t = 0; t < 5; ++t) o[qt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  bf16x8 ones;
#pragma unroll
  for (int j = 0; j < 8; ++j) ones[j] = f2bf(1.0f);
  int klim[QT];  // per query tile: this lane's query sees keys < klim
  int kmin[QT];  // ... and the smallest limit over the wave (wave-uniform)
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    klim[qt] = key_limit(p.mask_kind, qw + qt * 16 + col, p.sk, p.prefix_len);
    int t = klim[qt];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) t = min(t, __shfl_xor(t, o, 64));
    kmin[qt] = __builtin_amdgcn_readfirstlane(t);
  }
  const float c = p.scale_log2;
  // running maximum, the rescale threshold m_run * c + 8 and the exponent
  // offset -(m_run * c) (0 while every score so far was masked)
  float m_run[QT], m_thr[QT], m_off[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    m_run[qt] = -INFINITY;
    m_thr[qt] = -INFINITY * c + 8.f;
    m_off[qt] = -(0.f * c);
  }

  auto compute = [&](auto SI, int blk) {
    constexpr int S = decltype(SI)::value;
    const bf16* sk = S == 0 ? sK0 : S == 1 ? sK1 : sK2;
    const bf16* sv = S == 0 ? sV0 : S == 1 ? sV1 : sV2;
    const bf16* sl = S == 0 ? sL0 : S == 1 ? sL1 : sL2;
    const int k0 = blk * BKEY;
    // S^T: 4 key subtiles x 2 query tiles, K fragments shared by both
    f32x4 sacc[4][QT];
#pragma unroll
    for (int ts = 0; ts < 4; ++ts) {
      bf16x8 kf[2], klf[LO == 2 ? 2 : 1];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        kf[ks] = *reinterpret_cast<const bf16x8*>(&sk[kv_off(ts * 16 + col, ks * 32 + grp * 8)]);
        if constexpr (LO == 2)
          klf[ks] = *reinterpret_cast<const bf16x8*>(&sl[kv_off(ts * 16 + col, ks * 32 + grp * 8)]);
      }
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          if constexpr (LO == 2)
            a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(klf[ks], qf[qt][ks], a, 0, 0, 0);
          if constexpr (LO >= 1)
            a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[ks], qlf[qt][ks], a, 0, 0, 0);
          a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[ks], qf[qt][ks], a, 0, 0, 0);
        }
        sacc[ts][qt] = a;
      }
    }
    // online softmax per query tile (lane-local statistics)
    bf16x8 pf[QT][2];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      // only a block reaching past some query's limit needs the mask
      if (!FULL && k0 + BKEY > kmin[qt]) {
#pragma unroll
        for (int ts = 0; ts < 4; ++ts)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int kj = k0 + ts * 16 + grp * 4 + i;
            sacc[ts][qt][i] = kj < klim[qt] ? sacc[ts][qt][i] : -INFINITY;
          }
      }
      float mx = sacc[0][qt][0];
#pragma unroll
      for (int ts = 0; ts < 4; ++ts)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = smax(mx, sacc[ts][qt][i]);
      mx = max_xor32(max_xor16(mx));
      // Lazy rescaling: the running maximum moves only when some query of
      // the wave sees a score more than 2^8 (in exp2 units) above it; until
      // then the exponentials are taken against the stale maximum (values up
      // to 256, rounded to bf16 with the same relative error as values <= 1)
      // and the output / sum rescale is skipped for the whole wave.
      // (the threshold m_run * c + 8 and the exponent offset are updated only
      // when the maximum moves)
      const bool grow = mx * c > m_thr[qt];  // false while everything is masked
      if (__builtin_amdgcn_ballot_w64(grow)) {
        const float m_new = smax(m_run[qt], mx);
        const float alpha = m_run[qt] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((m_run[qt] - m_new) * c);
#pragma unroll
        for (int t = 0; t < 5; ++t) o[qt][t] *= alpha;
        m_run[qt] = m_new;
        m_thr[qt] = m_new * c + 8.f;
        m_off[qt] = -((m_new == -INFINITY ? 0.f : m_new) * c);  // fully-masked-so-far guard
      }
    }
    // O^T[d, q] += V^T[d, keys] . P^T[keys, q]; V^T fragments shared by every
    // query tile.  Each tile's probabilities for a 32-key half are computed
    // right before its MFMAs, so the exponentials of one tile overlap the
    // MFMAs of the one before.
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      bf16x8 vf[4];
#pragma unroll
      for (int td = 0; td < 4; ++td) {
        const v4i16 lo = v_tr_read(sv, kk * 32 + 4 * grp, td * 16, col);
        const v4i16 hi = v_tr_read(sv, kk * 32 + 16 + 4 * grp, td * 16, col);
        const v4i16 w8[2] = {lo, hi};
        vf[td] = *reinterpret_cast<const bf16x8*>(w8);
      }
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            pf[qt][kk][h * 4 + i] =
                f2bf(__builtin_amdgcn_exp2f(__builtin_fmaf(sacc[2 * kk + h][qt][i], c, m_off[qt])));
#pragma unroll
        for (int td = 0; td < 4; ++td)
          o[qt][td] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[td], pf[qt][kk], o[qt][td], 0, 0, 0);
        o[qt][4] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pf[qt][kk], o[qt][4], 0, 0, 0);
      }
    }
  };

  // ---- exact two-pass softmax (LO > 0) ----
  // scores of one block for every query tile, masked
  auto scores = [&](const bf16* sk, const bf16* sl, int k0, f32x4 (&sacc)[4][QT]) {
#pragma unroll
    for (int ts = 0; ts < 4; ++ts) {
      bf16x8 kf[2], klf[LO == 2 ? 2 : 1];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        kf[ks] = *reinterpret_cast<const bf16x8*>(&sk[kv_off(ts * 16 + col, ks * 32 + grp * 8)]);
        if constexpr (LO == 2)
          klf[ks] = *reinterpret_cast<const bf16x8*>(&sl[kv_off(ts * 16 + col, ks * 32 + grp * 8)]);
      }
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          if constexpr (LO == 2)
            a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(klf[ks], qf[qt][ks], a, 0, 0, 0);
          if constexpr (LO >= 1)
            a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[ks], qlf[qt][ks], a, 0, 0, 0);
          a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[ks], qf[qt][ks], a, 0, 0, 0);
        }
        sacc[ts][qt] = a;
      }
    }
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      if (k0 + BKEY > kmin[qt]) {
#pragma unroll
        for (int ts = 0; ts < 4; ++ts)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int kj = k0 + ts * 16 + grp * 4 + i;
            sacc[ts][qt][i] = kj < klim[qt] ? sacc[ts][qt][i] : -INFINITY;
          }
      }
    }
  };
  // pass 1: running maximum and the fp32 sum of exp(s - m), rescaled as the
  // maximum moves (m_run, l_run per query tile)
  float l_run[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) l_run[qt] = 0.f;
  auto stats = [&](auto SI, int blk) {
    constexpr int S = decltype(SI)::value;
    const bf16* sk = S == 0 ? sK0 : S == 1 ? sK1 : sK2;
    const bf16* sl = S == 0 ? sL0 : S == 1 ? sL1 : sL2;
    f32x4 sacc[4][QT];
    scores(sk, sl, blk * BKEY, sacc);
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      float mx = sacc[0][qt][0];
#pragma unroll
      for (int ts = 0; ts < 4; ++ts)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = smax(mx, sacc[ts][qt][i]);
      mx = max_xor32(max_xor16(mx));
      const float m_new = smax(m_run[qt], mx);
      const float off = -((m_new == -INFINITY ? 0.f : m_new) * c);
      const float alpha = m_run[qt] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(__builtin_fmaf(m_run[qt], c, off));
      float sum = 0.f;
#pragma unroll
      for (int ts = 0; ts < 4; ++ts)
#pragma unroll
        for (int i = 0; i < 4; ++i) sum += __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[ts][qt][i], c, off));
      sum = sum_xor32(sum_xor16(sum));
      l_run[qt] = __builtin_fmaf(l_run[qt], alpha, sum);
      m_run[qt] = m_new;
      m_off[qt] = off;
    }
  };
  // pass 2: p = bf16(exp(s - m) * (1 / l)), O^T += V^T . P^T
  float rl[QT];
  auto accum = [&](auto SI, int blk) {
    constexpr int S = decltype(SI)::value;
    const bf16* sk = S == 0 ? sK0 : S == 1 ? sK1 : sK2;
    const bf16* sv = S == 0 ? sV0 : S == 1 ? sV1 : sV2;
    const bf16* sl = S == 0 ? sL0 : S == 1 ? sL1 : sL2;
    f32x4 sacc[4][QT];
    scores(sk, sl, blk * BKEY, sacc);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      bf16x8 vf[4];
#pragma unroll
      for (int td = 0; td < 4; ++td) {
        const v4i16 lo = v_tr_read(sv, kk * 32 + 4 * grp, td * 16, col);
        const v4i16 hi = v_tr_read(sv, kk * 32 + 16 + 4 * grp, td * 16, col);
        const v4i16 w8[2] = {lo, hi};
        vf[td] = *reinterpret_cast<const bf16x8*>(w8);
      }
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        bf16x8 pf;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            pf[h * 4 + i] = f2bf(__builtin_amdgcn_exp2f(
                                     __builtin_fmaf(sacc[2 * kk + h][qt][i], c, m_off[qt])) *
                                 rl[qt]);
#pragma unroll
        for (int td = 0; td < 4; ++td)
          o[qt][td] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[td], pf, o[qt][td], 0, 0, 0);
      }
    }
  };

  // Before each barrier: s_waitcnt vmcnt(4) lgkmcnt(0) (vmcnt(6) with the K
  // remainders).  vmcnt: a stage is 4 (6) DMA instructions per wave and the
  // next stage stays in flight.
  // lgkmcnt(0): this wave's LDS reads of the stage computed before the
  // barrier have completed, since the DMA issued right after the barrier
  // refills that stage (the compiler would otherwise wait only at the reads'
  // first use, after the refill's issue).  gfx9 encoding, expcnt unconstrained.
  constexpr int kWaitOne = 0x070 | (LO == 2 ? 6 : 4);
  auto sync_step = [&]() __attribute__((always_inline)) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(kWaitOne);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  // Q is needed by every block: wait for it here, before the DMA prologue,
  // so the compiler has no pending load to drain at the loop entry
  __builtin_amdgcn_s_waitcnt(0xF70);
  // masked / ragged kernel (short key ranges: the expert's 50 or 241 keys):
  // after the last block, leave at once (nb is uniform across the
  // workgroup), with no further refills of never-read blocks and no further
  // barrier rounds.  (The same exits in the FULL kernel measured 6-7% slower
  // on the ViT's 16-block loop, so that loop keeps its original form.)
  auto ring = [&](auto&& comp) __attribute__((always_inline)) {
    issue(I0{}, 0);
    issue(I1{}, 1);
    for (int blk = 0; blk < nb; blk += 3) {
      sync_step();
      issue(I2{}, blk + 2);
      comp(I0{}, blk);
      if (!FULL && blk + 1 >= nb) break;
      sync_step();
      issue(I0{}, blk + 3);
      if (blk + 1 < nb) comp(I1{}, blk + 1);
      if (!FULL && blk + 2 >= nb) break;
      sync_step();
      issue(I1{}, blk + 4);
      if (blk + 2 < nb) comp(I2{}, blk + 2);
    }
  };
  if constexpr (LO > 0) {
    ring(stats);
    // every DMA landed and every wave's reads of the ring done before the
    // second pass refills it from block 0
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) rl[qt] = 1.0f / l_run[qt];
    ring(accum);
  } else {
    ring(compute);
  }
  // drain the trailing (never read) DMA before the workgroup exits
  __builtin_amdgcn_s_waitcnt(0);

#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int qi = qw + qt * 16 + col;
    if (qi >= p.sq) continue;
    const float l = o[qt][4][0];
    // (the exact two-pass form already normalised its probabilities)
    const float inv = LO > 0 ? 1.0f : l > 0.f ? 1.0f / l : 0.f;
    bf16* orow = p.o + b * p.o_bs + (long)qi * p.ldo + h * D;
#pragma unroll
    for (int td = 0; td < 4; ++td) {
      bf16x4 r;
#pragma unroll
      for (int i = 0; i < 4; ++i) r[i] = f2bf(o[qt][td][i] * inv);
      *reinterpret_cast<bf16x4*>(orow + td * 16 + grp * 4) = r;
    }
  }
}

// Exact attention for short key ranges (sk <= 64 NB: the RoPE'd layers' 50
// and 241 keys), single pass: the K rows (and their remainders, LO == 2) and
// V rows of the (sample, KV head) are staged into LDS once, every score of a
// query stays in registers (NB blocks x 4 subtiles), so the maximum, the fp32
// sum l = sum exp(s - m) and p = bf16(exp(s - m) * (1 / l)) -- torch's
// softmax(...).to(bf16) -- come without a second pass over K.  Wave w of the
// workgroup takes query tile (16 rows) blockIdx.x * qtiles + w % qtiles of
// head blockIdx.y * hpw + w / qtiles; the hpw heads share one KV head, whose
// K / V are then staged once for all of them.  LO as for attention_kernel
// (1: Q = q + q_lo; 2: also K = k + k_lo).
constexpr int SHORT_KEYS = 256;
template <int LO, int NB>
__global__ __launch_bounds__(1024, 1) void attention_short_kernel(AttnArgs p, int hpw, int qtiles) {
  constexpr int KLO = LO == 2 ? NB * BKEY * D : 64;
  __shared__ __attribute__((aligned(1024))) bf16 sK[NB * BKEY * D];
  __shared__ __attribute__((aligned(1024))) bf16 sV[NB * BKEY * D];
  __shared__ __attribute__((aligned(1024))) bf16 sL[KLO];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nw = blockDim.x >> 6;
  const int h = blockIdx.y * hpw + wave / qtiles, b = blockIdx.z;
  const int kvh = blockIdx.y * hpw * p.hkv / p.hq;
  const int q0 = blockIdx.x * qtiles * 16;
  const int grp = lane >> 4, col = lane & 15;
  const int qi = q0 + (wave % qtiles) * 16 + col;           // this lane's query row

  // keys any row of this workgroup may see
  int kend = p.sk;
  if (p.mask_kind != SVLA_MASK_NONE) {
    int lim = min(p.sq, q0 + qtiles * 16);
    if (p.mask_kind == SVLA_MASK_PREFIX_LM) lim = max(lim, p.prefix_len);
    kend = min(kend, lim);
  }
  const int nb = (kend + BKEY - 1) / BKEY;                   // <= NB (launcher)

  // stage K (+ K_lo) and V rows 0 .. 64 nb - 1 (clamped to sk - 1): one 1 KB
  // DMA instruction per 8 rows, dealt round the waves; chunk c of key row r
  // at slot c ^ (r & 7) (kv_off)
  {
    const bf16* kb = p.k + b * p.k_bs + kvh * D;
    const bf16* vb = p.v + b * p.v_bs + kvh * D;
    const bf16* lb = LO == 2 ? p.k_lo + b * p.k_bs + kvh * D : nullptr;
    const int n8 = nb * (BKEY / 8);
    for (int i = wave; i < n8; i += nw) {
      const int key = i * 8 + (lane >> 3);
      const int c = (lane & 7) ^ (key & 7);
      const long kr = min(key, p.sk - 1);
      __builtin_amdgcn_global_load_lds((void*)(kb + kr * p.ldk + c * 8), (lds_ptr_t)(sK + i * 512), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((void*)(vb + kr * p.ldv + c * 8), (lds_ptr_t)(sV + i * 512), 16, 0, 0);
      if constexpr (LO == 2)
        __builtin_amdgcn_global_load_lds((void*)(lb + kr * p.ldk + c * 8), (lds_ptr_t)(sL + i * 512), 16, 0, 0);
    }
  }
  // Q fragments (B operand of S^T), rows clamped (never stored past sq)
  const int qc = min(qi, p.sq - 1);
  const long qoff = b * p.q_bs + h * D + (long)qc * p.ldq;
  bf16x8 qf[2], qlf[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    qf[ks] = ld8(p.q + qoff + ks * 32 + grp * 8);
    if constexpr (LO >= 1) qlf[ks] = ld8(p.q_lo + qoff + ks * 32 + grp * 8);
  }
  const int klim = key_limit(p.mask_kind, qi, p.sk, p.prefix_len);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // S^T for every key block: s[blk][ts] lane holds keys 64 blk + 16 ts + 4 grp + i
  f32x4 s[NB][4];
#pragma unroll
  for (int blk = 0; blk < NB; ++blk)
#pragma unroll
    for (int ts = 0; ts < 4; ++ts) {
      f32x4 a = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
      if (blk < nb) {  // uniform
        a = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const int off = kv_off(blk * BKEY + ts * 16 + col, ks * 32 + grp * 8);
          const bf16x8 kf = *reinterpret_cast<const bf16x8*>(&sK[off]);
          if constexpr (LO == 2)
            a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*reinterpret_cast<const bf16x8*>(&sL[off]),
                                                        qf[ks], a, 0, 0, 0);
          if constexpr (LO >= 1) a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qlf[ks], a, 0, 0, 0);
          a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[ks], a, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (blk * BKEY + ts * 16 + grp * 4 + i >= klim) a[i] = -INFINITY;
      }
      s[blk][ts] = a;
    }
  const float c = p.scale_log2;
  float mx = s[0][0][0];
#pragma unroll
  for (int blk = 0; blk < NB; ++blk)
#pragma unroll
    for (int ts = 0; ts < 4; ++ts)
#pragma unroll
      for (int i = 0; i < 4; ++i) mx = smax(mx, s[blk][ts][i]);
  mx = max_xor32(max_xor16(mx));                   // finite: key 0 is always visible
  const float off = -(mx * c);
  float l = 0.f;
#pragma unroll
  for (int blk = 0; blk < NB; ++blk)
#pragma unroll
    for (int ts = 0; ts < 4; ++ts)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(s[blk][ts][i], c, off));
        s[blk][ts][i] = e;
        l += e;
      }
  l = sum_xor32(sum_xor16(l));
  const float rl = 1.0f / l;
  // O^T[d, q] += V^T[d, keys] . P^T[keys, q], p = bf16(e / l)
  f32x4 o[4];
#pragma unroll
  for (int td = 0; td < 4; ++td) o[td] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int blk = 0; blk < NB; ++blk) {
    if (blk >= nb) break;  // uniform
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      bf16x8 pf;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int i = 0; i < 4; ++i) pf[hh * 4 + i] = f2bf(s[blk][2 * kk + hh][i] * rl);
#pragma unroll
      for (int td = 0; td < 4; ++td) {
        const v4i16 lo = v_tr_read(sV, blk * BKEY + kk * 32 + 4 * grp, td * 16, col);
        const v4i16 hi = v_tr_read(sV, blk * BKEY + kk * 32 + 16 + 4 * grp, td * 16, col);
        const v4i16 w8[2] = {lo, hi};
        o[td] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*reinterpret_cast<const bf16x8*>(w8), pf,
                                                        o[td], 0, 0, 0);
      }
    }
  }
  if (qi >= p.sq) return;
  bf16* orow = p.o + b * p.o_bs + (long)qi * p.ldo + h * D;
#pragma unroll
  for (int td = 0; td < 4; ++td) {
    bf16x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = f2bf(o[td][i]);
    *reinterpret_cast<bf16x4*>(orow + td * 16 + grp * 4) = r;
  }
}

}  // namespace

extern "C" int svla_attention_lo_bf16(const void* q, const void* q_lo, int ldq, long q_bs,
                                      const void* k, const void* k_lo, int ldk, long k_bs,
                                      const void* v, int ldv, long v_bs, void* o, int ldo,
                                      long o_bs, int batch, int sq, int sk, int hq, int hkv,
                                      int head_dim, float scale, int mask_kind, int prefix_len,
                                      svla_stream_t stream) {
  if (head_dim != D || hq <= 0 || hkv <= 0 || hq % hkv || sq < 0 || sk <= 0 || batch < 0)
    return SVLA_EINVAL;
  if (mask_kind < SVLA_MASK_NONE || mask_kind > SVLA_MASK_PREFIX_LM) return SVLA_EINVAL;
  if (ldq % 8 || ldk % 8 || ldv % 8 || ldo % 4 || q_bs % 8 || k_bs % 8 || v_bs % 8 || o_bs % 4)
    return SVLA_EINVAL;
  if (ldq < hq * D || ldk < hkv * D || ldv < hkv * D || ldo < hq * D) return SVLA_EINVAL;
  if (!svla_aligned16(q) || !svla_aligned16(k) || !svla_aligned16(v) || ((uintptr_t)o & 7))
    return SVLA_EINVAL;
  if ((q_lo && !svla_aligned16(q_lo)) || (k_lo && !svla_aligned16(k_lo)) || (k_lo && !q_lo))
    return SVLA_EINVAL;
  if (sq == 0 || batch == 0) return SVLA_OK;
  AttnArgs p;
  p.q = static_cast<const bf16*>(q); p.ldq = ldq; p.q_bs = q_bs;
  p.k = static_cast<const bf16*>(k); p.ldk = ldk; p.k_bs = k_bs;
  p.q_lo = static_cast<const bf16*>(q_lo);
  p.k_lo = static_cast<const bf16*>(k_lo);
  p.v = static_cast<const bf16*>(v); p.ldv = ldv; p.v_bs = v_bs;
  p.o = static_cast<bf16*>(o); p.ldo = ldo; p.o_bs = o_bs;
  p.sq = sq; p.sk = sk; p.hq = hq; p.hkv = hkv;
  p.scale_log2 = scale * 1.4426950408889634f;
  p.mask_kind = mask_kind;
  p.prefix_len = prefix_len;
  const int lo = k_lo ? 2 : q_lo ? 1 : 0;
  // 16 query rows per wave (64 per workgroup) for short query ranges and for
  // grids that would leave the CUs with about one 128-row workgroup each;
  // 32 rows per wave (K / V LDS reads shared by two query tiles) otherwise,
  // and 64 (four query tiles share every K and V^T fragment read: 231 VGPRs,
  // two waves per SIMD) for unmasked grids of at least two 256-row
  // workgroups per CU, measured on MI355X: the batch-32 ViT attention (96
  // images x 12 heads x 1024 tokens) 531 -> 485 us in the same run,
  // bit-identical (each 16-query tile takes the same steps in every form).
  // Q / K remainders (RoPE'd layers: masked or short-key ranges) take the
  // checked kernel with 16 rows per wave (with 32 the remainder fragments
  // push it past 256 VGPRs).
  const long g2 = (long)((sq + BQ<2> - 1) / BQ<2>) * hq * batch;
  const long g4 = (long)((sq + BQ<4> - 1) / BQ<4>) * hq * batch;
  const bool qt1 = sq <= BQ<1> || g2 < 2 * kAttnCUs || lo > 0;
  const bool full = mask_kind == SVLA_MASK_NONE && sk % BKEY == 0 && lo == 0;
  hipStream_t s = (hipStream_t)stream;
  if (lo > 0 && sk <= SHORT_KEYS) {
    // RoPE'd layers: the single-pass exact form, one query head per
    // workgroup (the kernel can also give a KV group's hpw query heads one
    // workgroup that stages their K / V once; one head each measured as fast
    // or faster on MI355X, bit-identical: the expert's 50 x 241 cross
    // attention at batch 32 10.8 / 10.9 us, batch 1 9.4 -> 6.5 us; 50 x 50
    // self attention at batch 32 6.2 -> 5.3 us, batch 1 5.5 -> 4.0 us).  Up
    // to 16 query tiles (256 rows) per workgroup, fewer (down to 4) while
    // the grid has under 128 workgroups, each workgroup then staging the
    // head's K / V for its own query tiles (prefix 241 x 241, 15 / 5 heads:
    // batch 1 12.7 -> 7.2 us with 4 tiles, 60 workgroups; batch 2 12.9 ->
    // 7.5 us; batch 32 keeps 16: 35.7 us against 43.9 with 8).
    const int tiles = (sq + 15) / 16;
    const int hpw = 1;
    int qtiles = min(tiles, 16);
    while (qtiles > 4 && (long)((tiles + qtiles - 1) / qtiles) * hq * batch < 128) qtiles /= 2;
    dim3 grid((tiles + qtiles - 1) / qtiles, hq / hpw, batch);
    const dim3 block(64 * hpw * qtiles);
    if (sk <= BKEY) {
      if (lo == 1) hipLaunchKernelGGL((attention_short_kernel<1, 1>), grid, block, 0, s, p, hpw, qtiles);
      else hipLaunchKernelGGL((attention_short_kernel<2, 1>), grid, block, 0, s, p, hpw, qtiles);
    } else {
      if (lo == 1) hipLaunchKernelGGL((attention_short_kernel<1, 4>), grid, block, 0, s, p, hpw, qtiles);
      else hipLaunchKernelGGL((attention_short_kernel<2, 4>), grid, block, 0, s, p, hpw, qtiles);
    }
    SVLA_CHECK_LAUNCH();
    return SVLA_OK;
  }
  if (qt1) {
    dim3 grid((sq + BQ<1> - 1) / BQ<1>, hq, batch);
    if (full) hipLaunchKernelGGL((attention_kernel<true, 1, 0>), grid, dim3(256), 0, s, p);
    else if (lo == 0) hipLaunchKernelGGL((attention_kernel<false, 1, 0>), grid, dim3(256), 0, s, p);
    else if (lo == 1) hipLaunchKernelGGL((attention_kernel<false, 1, 1>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((attention_kernel<false, 1, 2>), grid, dim3(256), 0, s, p);
  } else if (full && g4 >= 2 * kAttnCUs) {
    dim3 grid((sq + BQ<4> - 1) / BQ<4>, hq, batch);
    hipLaunchKernelGGL((attention_kernel<true, 4, 0>), grid, dim3(256), 0, s, p);
  } else {
    dim3 grid((sq + BQ<2> - 1) / BQ<2>, hq, batch);
    if (full) hipLaunchKernelGGL((attention_kernel<true, 2, 0>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((attention_kernel<false, 2, 0>), grid, dim3(256), 0, s, p);
  }
  SVLA_CHECK_LAUNCH();
  return SVLA_OK;
}

extern "C" int svla_attention_bf16(const void* q, int ldq, long q_bs, const void* k, int ldk,
                                   long k_bs, const void* v, int ldv, long v_bs, void* o, int ldo,
                                   long o_bs, int batch, int sq, int sk, int hq, int hkv,
                                   int head_dim, float scale, int mask_kind, int prefix_len,
                                   svla_stream_t stream) {
  return svla_attention_lo_bf16(q, nullptr, ldq, q_bs, k, nullptr, ldk, k_bs, v, ldv, v_bs, o,
                                ldo, o_bs, batch, sq, sk, hq, hkv, head_dim, scale, mask_kind,
                                prefix_len, stream);
}
