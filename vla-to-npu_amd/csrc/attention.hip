// Fused grouped-query attention for gfx950 (head_dim 64).
//
// Replaces the reference's per-head chain  score GEMM -> (masked) softmax ->
// P.V GEMM  (vla/text_encoder_bf16.py:502-526, vla/vision_block_bf16.py:325-367,
// vla/action_expert_bf16.py:689-713, 764-787) with one kernel per call.
// Numerics follow the torch modules (vla/text_encoder_bf16.py:117-126):
// scores and softmax statistics in fp32, probabilities rounded to bf16 before
// the P.V product, fp32 accumulation, bf16 output.
//
// Work decomposition: one workgroup = 64 query rows of one query head
// (4 waves x 16 rows); the loop runs over blocks of 64 keys of the head's KV
// group (h * hkv / hq), staged in LDS and shared by the 4 waves.
//
// MFMA layout trick: every product is computed transposed,
//   S^T[key, q] = K . Q^T         (A = K tile from LDS, B = the wave's Q rows)
//   O^T[d, q]  += V^T . P^T       (A = V^T tile from LDS, B = P^T from registers)
// With v_mfma_f32_16x16x32_bf16 the accumulator of lane l holds 4 consecutive
// rows of column (l & 15); transposing puts the QUERY on the column, so each
// lane owns one query's scores, running max, running sum and output -- the
// online-softmax rescale is lane-local and the row reductions are two
// cross-lane shuffles (lanes l, l^16, l^32).  The S^T accumulators of two
// consecutive 16-key subtiles are exactly the B operand P^T of the next MFMA
// (keys {4g..4g+3} u {16+4g..16+4g+3} in k-slots 8g..8g+7); the V^T operand is
// read with the same key permutation, so no shuffles are needed between the
// two products.
#include "svla_common.h"

namespace {

constexpr int D = 64;
constexpr int BQ = 64;     // query rows per workgroup
constexpr int BKEY = 64;   // keys per LDS block
constexpr int KS = D + 8;  // padded LDS row (elements) for the K tile
constexpr int VS = BKEY + 8;

struct AttnArgs {
  const bf16* q; long ldq, q_bs;
  const bf16* k; long ldk, k_bs;
  const bf16* v; long ldv, v_bs;
  bf16* o; long ldo, o_bs;
  int sq, sk, hq, hkv;
  float scale_log2;  // scale * log2(e)
  int mask_kind, prefix_len;
};

__device__ __forceinline__ bool masked(int kind, int qi, int kj, int prefix_len) {
  if (kind == SVLA_MASK_CAUSAL) return kj > qi;
  if (kind == SVLA_MASK_PREFIX_LM) return kj > qi && kj >= prefix_len;
  return false;
}

__global__ __launch_bounds__(256) void attention_kernel(AttnArgs p) {
  __shared__ __attribute__((aligned(16))) bf16 sK[BKEY * KS];
  __shared__ __attribute__((aligned(16))) bf16 sVt[D * VS];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = blockIdx.y, b = blockIdx.z;
  const int g = h * p.hkv / p.hq;
  const int q0 = blockIdx.x * BQ;
  const int qi = q0 + wave * 16 + (lane & 15);  // this lane's query row
  const int grp = lane >> 4;                     // 0..3

  const bf16* qb = p.q + b * p.q_bs + h * D;
  const bf16* kb = p.k + b * p.k_bs + g * D;
  const bf16* vb = p.v + b * p.v_bs + g * D;

  // B operand of S^T: Q[qi][ks*32 + 8*grp .. +7]
  bf16x8 qf[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
    qf[ks] = qi < p.sq ? ld8(qb + (long)qi * p.ldq + ks * 32 + grp * 8) : bf16x8{};

  // last key any row of this workgroup may see
  int kend = p.sk;
  if (p.mask_kind != SVLA_MASK_NONE) {
    const int qmax = min(p.sq, q0 + BQ) - 1;
    int lim = qmax + 1;
    if (p.mask_kind == SVLA_MASK_PREFIX_LM) lim = max(lim, p.prefix_len);
    kend = min(kend, lim);
  }

  f32x4 o[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  for (int k0 = 0; k0 < kend; k0 += BKEY) {
    // stage K [64 keys][64 d] and V^T [64 d][64 keys]
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = tid + i * 256;
      const int key = c >> 3, dc = (c & 7) * 8;
      const int kj = k0 + key;
      bf16x8 kv = kj < p.sk ? ld8(kb + (long)kj * p.ldk + dc) : bf16x8{};
      bf16x8 vv = kj < p.sk ? ld8(vb + (long)kj * p.ldv + dc) : bf16x8{};
      *reinterpret_cast<bf16x8*>(&sK[key * KS + dc]) = kv;
#pragma unroll
      for (int j = 0; j < 8; ++j) sVt[(dc + j) * VS + key] = vv[j];
    }
    __syncthreads();

    // S^T for 4 subtiles of 16 keys
    float s[4][4];
#pragma unroll
    for (int ts = 0; ts < 4; ++ts) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const bf16x8 kf =
            *reinterpret_cast<const bf16x8*>(&sK[(ts * 16 + (lane & 15)) * KS + ks * 32 + grp * 8]);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[ks], acc, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kj = k0 + ts * 16 + grp * 4 + i;
        const bool dead = kj >= p.sk || masked(p.mask_kind, qi, kj, p.prefix_len);
        s[ts][i] = dead ? -INFINITY : acc[i] * p.scale_log2;
      }
    }
    // row max over this block: 16 local values, then lanes l, l^16, l^32, l^48
    float mx = s[0][0];
#pragma unroll
    for (int ts = 0; ts < 4; ++ts)
#pragma unroll
      for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[ts][i]);
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;  // fully-masked-so-far guard
    const float alpha = exp2f(m_run - m_use);
    float psum = 0.f;
    bf16x8 pf[2];
#pragma unroll
    for (int ts = 0; ts < 4; ++ts)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float e = exp2f(s[ts][i] - m_use);
        psum += e;
        pf[ts >> 1][(ts & 1) * 4 + i] = f2bf(e);
      }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int t = 0; t < 4; ++t) o[t] *= alpha;

    // O^T[d, q] += V^T[d, keys] . P^T[keys, q]
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
      for (int td = 0; td < 4; ++td) {
        const bf16* vrow = &sVt[(td * 16 + (lane & 15)) * VS + kk * 32 + grp * 4];
        const bf16x4 lo = *reinterpret_cast<const bf16x4*>(vrow);
        const bf16x4 hi = *reinterpret_cast<const bf16x4*>(vrow + 16);
        bf16x8 vf;
        vf[0] = lo[0]; vf[1] = lo[1]; vf[2] = lo[2]; vf[3] = lo[3];
        vf[4] = hi[0]; vf[5] = hi[1]; vf[6] = hi[2]; vf[7] = hi[3];
        o[td] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf[kk], o[td], 0, 0, 0);
      }
    }
    __syncthreads();
  }

  if (qi >= p.sq) return;
  const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
  bf16* orow = p.o + b * p.o_bs + (long)qi * p.ldo + h * D;
#pragma unroll
  for (int td = 0; td < 4; ++td) {
    bf16x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = f2bf(o[td][i] * inv);
    *reinterpret_cast<bf16x4*>(orow + td * 16 + grp * 4) = r;
  }
}

}  // namespace

extern "C" int svla_attention_bf16(const void* q, int ldq, long q_bs, const void* k, int ldk,
                                   long k_bs, const void* v, int ldv, long v_bs, void* o, int ldo,
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
  if (sq == 0 || batch == 0) return SVLA_OK;
  AttnArgs p;
  p.q = static_cast<const bf16*>(q); p.ldq = ldq; p.q_bs = q_bs;
  p.k = static_cast<const bf16*>(k); p.ldk = ldk; p.k_bs = k_bs;
  p.v = static_cast<const bf16*>(v); p.ldv = ldv; p.v_bs = v_bs;
  p.o = static_cast<bf16*>(o); p.ldo = ldo; p.o_bs = o_bs;
  p.sq = sq; p.sk = sk; p.hq = hq; p.hkv = hkv;
  p.scale_log2 = scale * 1.4426950408889634f;
  p.mask_kind = mask_kind;
  p.prefix_len = prefix_len;
  dim3 grid((sq + BQ - 1) / BQ, hq, batch);
  hipLaunchKernelGGL(attention_kernel, grid, dim3(256), 0, (hipStream_t)stream, p);
  SVLA_CHECK_LAUNCH();
  return SVLA_OK;
}
