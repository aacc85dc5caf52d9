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
//      l ^ 16 and l ^ 32 through permlane swaps) in fp32, base 2, scale folded in, with a lazy
//      rescale of the running output;
//   3. accumulates O^T += V^T P^T with the same MFMA: the lane's probabilities, rounded to bf16,
//      are already the B operand (8 keys per lane group: 4 from each of two 16-key blocks), and
//      A takes V^T rows over those same 8 keys from LDS. k order only has to agree between A and
//      B, so no shuffle of P is needed. The row sums of P come from the same MFMA with an
//      all-ones A operand (the matrix cores have slack; the vector ALUs do not).
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
// log2 of the largest probability the lazy rescale lets through before moving the reference
constexpr float kRescaleLog2 = 8.f;

typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));

// QB: 16-query blocks per wave (the workgroup takes 64 QB queries); each K and V^T fragment
// read from LDS feeds QB MFMAs.
template <int QB>
__device__ void flashAttention(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                               uint16_t* out, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk,
                               int causal, float scale_log2, int out_bshd) {
  constexpr int kTileQ = 64 * QB;
  __shared__ __attribute__((aligned(16))) uint16_t Ks[kTileK * kPitch];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[kD * kVPitch];
  const int t = threadIdx.x, lane = t % kWave, wave = t / kWave;
  const int r = lane % 16, g = lane / 16;
  // Workgroups are dispatched in linear-id order, and the query tile is the slow index of that
  // order, walked from the last tile (most keys under a causal mask) to the first: the longest
  // workgroups start first and the short ones fill in behind them. (With the tile as the fast
  // index, a long tile dispatched late set the kernel's end: 114 us against 67 us at 4 x 2048.)
  const uint64_t lin = blockIdx.x + static_cast<uint64_t>(gridDim.x) * blockIdx.y;
  const int64_t bh = lin % gridDim.y;  // b * Hq + h
  const int64_t b = bh / Hq, h = bh % Hq;
  const int64_t kvh = h / (Hq / Hkv);
  const int64_t q0 = static_cast<int64_t>(gridDim.x - 1 - lin / gridDim.y) * kTileQ;
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
  const uint16_t* kp = kbase + pair_key * kD + d0;
  const uint16_t* vp = vbase + pair_key * kD + d0;
  U128 kr[2], vr[2];
  auto fetch = [&](int64_t k0) {
    const uint16_t* kq = kp + k0 * kD;
    const uint16_t* vq = vp + k0 * kD;
    if (k0 + kTileK <= Sk) {  // uniform: every key of the tile exists
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        kr[u] = gload16(kq + u * kD);
        vr[u] = gload16(vq + u * kD);
      }
    } else {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const bool in = k0 + pair_key + u < Sk;
        kr[u] = in ? gload16(kq + u * kD) : zero16();
        vr[u] = in ? gload16(vq + u * kD) : zero16();
      }
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
  // row sums of the bf16 probabilities, as an MFMA against an all-ones A operand: every element
  // of lane (r, g) ends up holding the sum for query 16 qb + r (only element 0 is kept current)
  f32x4 lsum[QB];
  float m_run[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m_run[qb] = -INFINITY;
    lsum[qb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[qb][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const U128 ones{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};  // bf16 1.0 x 8

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
    // 2. online softmax per query (masked keys: -inf). The reference point is kept in scaled
    // units; max(s * c) = c * max(s) for the positive scale c, so each probability is one fma
    // and one v_exp_f32 (every argument <= kRescaleLog2 or -inf).
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
      // Lazy rescale: the reference point m_run moves only when a score passes it by more than
      // kRescaleLog2 (base 2), so probabilities stay below 2^kRescaleLog2 and the o / lsum
      // rescale runs on few tiles. The final o / l is unchanged by the choice of reference.
      // A query that has seen no key yet keeps m = -inf and probabilities 0.
      const float tm = tmax * scale_log2;
      const bool grow = tm > m_run[qb] + kRescaleLog2;  // false while tm = -inf
      if (__builtin_amdgcn_ballot_w64(grow)) {
        const float alpha = grow ? __builtin_amdgcn_exp2f(m_run[qb] - tm) : 1.f;  // 0 from -inf
        m_run[qb] = grow ? tm : m_run[qb];
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) o[qb][dt] *= alpha;
        lsum[qb][0] *= alpha;
      }
      const float base = m_run[qb] == -INFINITY ? 0.f : m_run[qb];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          s[qb][kk][i] = __builtin_amdgcn_exp2f(fmaf(s[qb][kk][i], scale_log2, -base));
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
#pragma unroll
    for (int kc = 0; kc < 2; ++kc)
#pragma unroll
      for (int qb = 0; qb < QB; ++qb)
        lsum[qb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(asBf16x8(ones), pb[qb][kc], lsum[qb],
                                                           0, 0, 0);
  }
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int64_t qi = qw + qb * 16 + r;
    if (qi >= Sq) continue;
    const float l = lsum[qb][0];
    const float inv = l > 0.f ? 1.f / l : 0.f;
    // out [B, Hq, Sq, D], or [B, Sq, Hq, D] (the layout the transpose after attention makes)
    uint16_t* orow = out + (out_bshd ? (b * Sq + qi) * Hq + h : bh * Sq + qi) * kD + g * 4;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const uint32_t lo = packBf16x2(o[qb][dt][0] * inv, o[qb][dt][1] * inv);
      const uint32_t hi = packBf16x2(o[qb][dt][2] * inv, o[qb][dt][3] * inv);
      *gp(reinterpret_cast<uint2*>(orow + dt * 16)) = uint2{lo, hi};
    }
  }
}

}  // namespace

// amdgpu_waves_per_eu(2) caps the kernels at 256 VGPRs, which makes the compiler pick the VGPR
// form of the MFMAs: in the AGPR form every tile moved the score and output accumulators through
// v_accvgpr_read / write (80 extra VALU instructions per tile). Grid: {ceil(Sq / (64 QB)), B Hq}.
//
// 16 queries per wave (64 per workgroup): short query sequences.
extern "C" __global__ void __launch_bounds__(kFlashThreads) __attribute__((amdgpu_waves_per_eu(2)))
    flash_attention_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* out,
                         int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk, int causal,
                         float scale_log2, int out_bshd) {
  flashAttention<1>(q, k, v, out, Hq, Hkv, Sq, Sk, causal, scale_log2, out_bshd);
}

// 32 queries per wave (128 per workgroup): each K and V^T fragment read from LDS feeds two MFMAs,
// and one staged tile serves twice the queries. 154 VGPRs, 3 waves per SIMD; at the Qwen2
// prefill size (4 x 2048 tokens, 14 / 2 heads, causal) 56 us against 67 us for the 16-query form.
extern "C" __global__ void __launch_bounds__(kFlashThreads) __attribute__((amdgpu_waves_per_eu(2)))
    flash_attention_bf16_q32(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                             uint16_t* out, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk,
                             int causal, float scale_log2, int out_bshd) {
  flashAttention<2>(q, k, v, out, Hq, Hkv, Sq, Sk, causal, scale_log2, out_bshd);
}
