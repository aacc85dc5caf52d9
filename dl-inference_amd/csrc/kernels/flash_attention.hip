// Flash-style attention for prefill on gfx950: softmax(q k^T * scale [+ causal mask]) v over
// contiguous bf16 [B, H, S, 64] q / k / v with grouped KV heads (attention/kernel.py:6-62; the
// same masking as attention.hip: with the causal flag, query i sees keys [0, Sk - Sq + i]).
//
// A 256-thread workgroup owns 64 QB queries of one (batch, q head); wave w owns 16 QB of them. Keys go
// by in tiles of 64: the workgroup stages K as [key][d] and V transposed as [d][key] in LDS (the
// next tile's loads are in flight while the current one is used), and each wave
//   1. scores the tile transposed, S^T = K Q^T, with v_mfma_f32_16x16x32_bf16 (A = 16 keys x 32 d
//      from LDS, B = 32 d x 16 queries from registers): lane l then holds the scores of query
//      l % 16 for keys 4 (l / 16) + i of each 16-key block;
//   2. runs the online softmax per query (a column of S^T: the lane's 16 values, then lanes
//      l ^ 16 and l ^ 32 through permlane swaps) in fp32, base 2, scale folded in;
//   3. accumulates O^T += V^T P^T with the same MFMA: the lane's probabilities, rounded to bf16,
//      are already the B operand (8 keys per lane group: 4 from each of two 16-key blocks), and
//      A takes V^T rows over those same 8 keys from LDS. k order only has to agree between A and
//      B, so no shuffle of P is needed.
// Query tiles are walked from the last (most keys under a causal mask) to the first.
#include "common.h"
#include "skinny.h"

using namespace dk;

namespace {

constexpr int kFlashThreads = 256;
constexpr int kD = 64;        // head dim
constexpr int kTileK = 64;    // keys per tile
constexpr int kPitch = 72;    // K row pitch in bf16 (144 bytes: 16-byte aligned rows)
// V^T row pitch in bf16 (136 bytes: 8-byte aligned for the fragment reads). The stash writes
// 4-byte words to rows d0 + j of 8 column groups d0 = 8m: at 34 words per row those rows start
// 16 banks apart (at 36 words, every other group landed on the same banks).
constexpr int kVPitch = 68;

typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));

// QB: 16-query blocks per wave (the workgroup takes 64 QB queries); each K and V^T fragment
// read from LDS feeds QB MFMAs.
template <int QB>
__device__ void flashAttention(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                               uint16_t* out, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk,
                               int causal, float scale_log2) {
  constexpr int kTileQ = 64 * QB;
  __shared__ __attribute__((aligned(16))) uint16_t Ks[kTileK * kPitch];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[kD * kVPitch];
  const int t = threadIdx.x, lane = t % kWave, wave = t / kWave;
  const int r = lane % 16, g = lane / 16;
  const int64_t bh = blockIdx.y;  // b * Hq + h
  const int64_t b = bh / Hq, h = bh % Hq;
  const int64_t kvh = h / (Hq / Hkv);
  const int64_t q0 = static_cast<int64_t>(gridDim.x - 1 - blockIdx.x) * kTileQ;
  const int64_t qw = q0 + wave * 16 * QB;  // the wave's first query
  const uint16_t* kbase = k + (b * Hkv + kvh) * Sk * kD;
  const uint16_t* vbase = v + (b * Hkv + kvh) * Sk * kD;
  const int64_t shift = Sk - Sq;

  // this lane's queries qw + 16 qb + r (clamped into range for the loads; results past Sq are
  // not stored) and the keys each may see
  U128 qf[QB][2];
  int lim32[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int64_t qi = qw + qb * 16 + r;
    const int64_t qrow = qi < Sq ? qi : Sq - 1;
    const uint16_t* qp = q + (bh * Sq + qrow) * kD + g * 8;
    qf[qb][0] = gload16(qp);
    qf[qb][1] = gload16(qp + 32);
    int64_t limit = causal ? shift + qi + 1 : Sk;
    lim32[qb] = static_cast<int>(limit < 0 ? 0 : (limit > Sk ? Sk : limit));
  }
  // keys any query of the workgroup sees, and keys every query of this wave sees (tiles below
  // that need no mask)
  int64_t wg_keys = causal ? shift + (q0 + kTileQ) : Sk;
  wg_keys = wg_keys < 0 ? 0 : (wg_keys > Sk ? Sk : wg_keys);
  int64_t wave_keys = causal ? shift + qw + 1 : Sk;
  wave_keys = wave_keys < 0 ? 0 : (wave_keys > Sk ? Sk : wave_keys);

  // staging: thread t moves the 16-byte chunks of keys 2 (t / 8) and 2 (t / 8) + 1 at columns
  // d0 = (t % 8) * 8 of the K tile and of the V tile. Two adjacent keys of the same columns let
  // the transposed V store write 4-byte words (keys 2p, 2p + 1 of one d).
  const int pair_key = 2 * (t / 8), d0 = (t % 8) * 8;
  U128 kr[2], vr[2];
  auto fetch = [&](int64_t k0) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int64_t key = k0 + pair_key + u;
      const int64_t off = key * kD + d0;
      kr[u] = key < Sk ? gload16(kbase + off) : zero16();
      vr[u] = key < Sk ? gload16(vbase + off) : zero16();
    }
  };
  auto stash = [&] {
#pragma unroll
    for (int u = 0; u < 2; ++u)
      *reinterpret_cast<U128*>(&Ks[(pair_key + u) * kPitch + d0]) = kr[u];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // vr[u][j] = (V[key u][d0 + 2j], V[key u][d0 + 2j + 1]) as lo | hi << 16
      const uint32_t even = (vr[0][j] & 0xFFFFu) | (vr[1][j] << 16);
      const uint32_t odd = (vr[0][j] >> 16) | (vr[1][j] & 0xFFFF0000u);
      *reinterpret_cast<uint32_t*>(&Vt[(d0 + 2 * j) * kVPitch + pair_key]) = even;
      *reinterpret_cast<uint32_t*>(&Vt[(d0 + 2 * j + 1) * kVPitch + pair_key]) = odd;
    }
  };

  f32x4 o[QB][4];  // O^T tiles: d = 16 dt + 4 g + i, query 16 qb + r
  float m_run[QB], l_run[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m_run[qb] = -INFINITY;
    l_run[qb] = 0.f;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[qb][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  const int tiles = static_cast<int>((wg_keys + kTileK - 1) / kTileK);
  if (tiles > 0) fetch(0);
  for (int kt = 0; kt < tiles; ++kt) {
    const int64_t k0 = static_cast<int64_t>(kt) * kTileK;
    __syncthreads();  // the previous tile is no longer read
    stash();
    __syncthreads();
    if (kt + 1 < tiles) fetch(k0 + kTileK);

    // 1. S^T for 4 blocks of 16 keys and each query block
    f32x4 s[QB][4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const uint16_t* krow = &Ks[(kk * 16 + r) * kPitch + g * 8];
      const U128 ka = *reinterpret_cast<const U128*>(krow);
      const U128 kb = *reinterpret_cast<const U128*>(krow + 32);
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        s[qb][kk] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(asBf16x8(ka), asBf16x8(qf[qb][0]),
                                                            f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        s[qb][kk] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(asBf16x8(kb), asBf16x8(qf[qb][1]),
                                                            s[qb][kk], 0, 0, 0);
      }
    }
    // 2. online softmax per query (masked keys: -inf). The running max is kept in scaled units;
    // max(s * c) = c * max(s) for the positive scale c, so each probability is one fma and one
    // v_exp_f32 (every argument <= 0 or -inf, results in [0, 1], no range reduction needed).
    const bool full = k0 + kTileK <= wave_keys;  // uniform over the wave: every key visible
    bf16x8 pb[QB][2];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      float tmax = -INFINITY;
      if (full) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
          for (int i = 0; i < 4; ++i) tmax = fmaxf(tmax, s[qb][kk][i]);
      } else {
        const int key0 = static_cast<int>(k0) + g * 4;  // lengths < 2^30 (host check)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float x = key0 + kk * 16 + i < lim32[qb] ? s[qb][kk][i] : -INFINITY;
            s[qb][kk][i] = x;
            tmax = fmaxf(tmax, x);
          }
      }
      tmax = rowsMax(tmax);  // over lanes r, r + 16, r + 32, r + 48: the query's 64 keys
      const float m_new = fmaxf(m_run[qb], tmax * scale_log2);
      // a query that has seen no key yet keeps m = -inf and probabilities 0
      const float base = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run[qb] - base);  // 0 while m_run = -inf
      float psum = 0.f;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pv = __builtin_amdgcn_exp2f(fmaf(s[qb][kk][i], scale_log2, -base));
          s[qb][kk][i] = pv;
          psum += pv;
        }
      l_run[qb] = l_run[qb] * alpha + rowsSum(psum);
      m_run[qb] = m_new;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) o[qb][dt] *= alpha;
      // keys of 32-key chunk kc, lane group g: 4 g + i of blocks 2 kc and 2 kc + 1
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const bf16x4_t lo = __builtin_convertvector(s[qb][2 * kc], bf16x4_t);
        const bf16x4_t hi = __builtin_convertvector(s[qb][2 * kc + 1], bf16x4_t);
        pb[qb][kc] = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
    }
    // 3. O^T += V^T P^T, 32 keys per MFMA; each V^T fragment serves every query block
#pragma unroll
    for (int kc = 0; kc < 2; ++kc)
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const uint16_t* vrow = &Vt[(dt * 16 + r) * kVPitch + kc * 32 + g * 4];
        const uint2 a0 = *reinterpret_cast<const uint2*>(vrow);
        const uint2 a1 = *reinterpret_cast<const uint2*>(vrow + 16);
        const U128 va{a0.x, a0.y, a1.x, a1.y};
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
          o[qb][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(asBf16x8(va), pb[qb][kc],
                                                              o[qb][dt], 0, 0, 0);
      }
  }
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int64_t qi = qw + qb * 16 + r;
    if (qi >= Sq) continue;
    const float inv = l_run[qb] > 0.f ? 1.f / l_run[qb] : 0.f;
    uint16_t* orow = out + (bh * Sq + qi) * kD + g * 4;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const uint32_t lo = packBf16x2(o[qb][dt][0] * inv, o[qb][dt][1] * inv);
      const uint32_t hi = packBf16x2(o[qb][dt][2] * inv, o[qb][dt][3] * inv);
      *gp(reinterpret_cast<uint2*>(orow + dt * 16)) = uint2{lo, hi};
    }
  }
}

}  // namespace

// 16 queries per wave. With QB = 2 (32 per wave, 128 per workgroup) the kernel needs 150 VGPRs,
// halving occupancy, and measured slower at the Qwen2 prefill size (140 us against 125 us).
extern "C" __global__ void __launch_bounds__(kFlashThreads)
    flash_attention_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* out,
                         int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk, int causal,
                         float scale_log2) {
  flashAttention<1>(q, k, v, out, Hq, Hkv, Sq, Sk, causal, scale_log2);
}
