// Training backward of the GDN-2 recurrence on gfx950.  fp32 mode runs every
// product on v_mfma_f32_16x16x4_f32; bf16 mode runs the state scans,
// k_bw_grads' products and k_bw_intra's W, U0, Xf and P products as split-bf16
// products (hi + lo words, three v_mfma_f32_16x16x32_bf16), the rest in fp32.  State, carries and
// accumulations are fp32 in both.
//
// Reference: the custom VJP of chunk_gdn2 (maelie-labs/deltanet-tpu v0.3.0,
// src/deltanet_tpu/gdn2.py:1446-1769) with its backward kernels
// (gdn2.py:243-493 analytical prepass adjoint, 496-582, 698-769 reverse state
// scan).  The recurrence differentiated is reference.py:123-161:
//   Sd = e^{g_t} S ; u = w v - Sd^T (b k) ; S' = Sd + k u^T ; o = S'^T q.
//
// Chunk form (C = 64 tokens, G_i = cumulative log-decay from the start of the
// chunk or of token i's document, whichever is later,
// carry_i = token i continues the state entering the chunk, last_j = token j
// is in the chunk's last document, same(i,j) = same document):
//   A_ij = sum_r b_i k_i[r] k_j[r] e^{G_i-G_j}  (j < i, same)   T = (I + A)^-1
//   M_ij = sum_r q_i[r] k_j[r] e^{G_i-G_j}      (j <= i, same)
//   W = T diag(carry) (b k e^G) ; U0 = T (w v) ; U = U0 - W S_c
//   Kc_j = last_j k_j e^{G_last-G_j} ; lam = all_carry e^{G_last}
//   Xf = diag(carry) q e^G - M W
//   S_{c+1} = lam * S_c + Kc^T U            O_c = Xf S_c + M U0
// and its adjoint, the same affine map transposed and run backwards:
//   dS_c = lam * dS_{c+1} + Xf^T dO_c - W^T (Kc dS_{c+1})
// plus the chunk-local parameter gradients (dU = M^T dO + Kc dS_{c+1},
// dX = T^T dU, dM = dO U^T, dA = -dX U^T, ...; see k_bw_grads).
//
// Every decay factor is formed as a product of factors <= 1: a pair (i, j)
// with j <= m <= i uses e^{G_i-G_m} e^{G_m-G_j}, m = the first row of i's
// 16-row block (or the last row of j's block); pairs inside one 16-row block
// use e^{G_i-G_j} directly.  No factor can overflow, whatever the decay
// (the reference's strong-decay test uses g = -150 per token).
//
// Kernels (one launch each, in stream order):
//   k_bw_intra   per (batch, head, chunk), persistent (one workgroup per CU
//                looping over the units): A, M, T, W, U0, Xf, Kc, lam, G and
//                the reverse scan's state-free term Xf^T dO
//   k_bw_chains  per (batch, head, block of 16 or 32 state columns) and
//                direction, both scans in one launch: forward S_c for every
//                chunk; reverse dS_{c+1} for every chunk, dS_0
//   k_bw_grads   per (batch, head, chunk): dv, dw, dM, dA, the chunk-wide
//                products of dq, dk, db and rowsum(S_c * dS_{c+1})
//   k_bw_dqk     per (batch, head, chunk, quarter of the key channels): dq, dk,
//                db, dg
#include "dn_common.h"
#include "dn_host.h"

namespace dn {

namespace {

constexpr int BC = 64;        // tokens per backward chunk
constexpr int KD = 128;       // K = V = 128
constexpr int CK = BC * KD;
constexpr int CC = BC * BC;
constexpr int KK = KD * KD;
constexpr int KP = KD + 4;    // padded LDS row pitch (128-wide rows)
constexpr int CP = BC + 4;    // padded LDS row pitch (64-wide rows)
constexpr int NWV = 8;        // waves per workgroup of the chunk-parallel kernels
constexpr int NT = 64 * NWV;
constexpr int TPW = 8 / NWV;  // 16-column tiles per wave in C x 128 products

struct BW {
  int B, L, H, NC;       // NC: chunks of this launch's token block
  int bf;                // precision "bf16": split-bf16 products in k_bw_grads
  int c0;                // first chunk of the block (token c0 * BC)
  const float *q, *k, *v, *g, *b, *w;
  int qk_hd, gb_hd;      // q, k (g, b) hold H / hd heads: head h reads head h / hd
  const int32_t* seg;
  const float* init;     // state entering the block's first chunk (NULL: zero)
  float* sfin;           // NULL or: the forward scan's state leaving the block
  const void* dout;      // cotangent of the output, element type dout_dt
  int dout_dt, dv_dt;    // DT_F32 or DT_BF16 (dv is written in dv_dt)
  int v_dt;              // element type of v (DT_F32 or DT_BF16)
  const float* dfin;     // gradient of the state leaving the block (NULL: zero)
  float *dq, *dk, *dv, *dg, *db, *dw;
  float* dinit;          // NULL or: the reverse scan's gradient of the state entering the block
  // workspace, per unit u = (batch * H + head) * NC + chunk
  float *G;    // [BC][KD] cumulative log2-decay from the chunk's or the token's document start
  float *Wm;   // [BC][KD] W          (these four in gofs / bofs order)
  float *WT;   // [KD][BC] W^T
  float *Kc;   // [BC][KD]
  float *KcT;  // [KD][BC]
  float *PT;   // [KD][KD] (Xf^T dO)^T, element (v, k) at aofs(v, k)
  float *U0T;  // [KD][BC] U0^T, aofs order
  float *MT;   // [BC][BC] M^T
  float *TT;   // [BC][BC] T^T
  float *lam;  // [KD]
  float *dMw, *dAw; // [BC][BC] dM and dA (k_bw_grads -> k_bw_dqk)
  float *RS;   // [KD] rowsum over v of S_c * dS_{c+1} per channel (k_bw_grads -> k_bw_dqk)
  float *Rq, *Rk, *Rb; // raw dO S0^T, U dSC^T, dX S0^T (k_bw_grads -> k_bw_dqk), in
                       // MFMA accumulator order: [column tile][row block][lane][4]
  float *S;         // [KD][KD] state entering the chunk, transposed: element (v, k) at v * KD + k
  float *dS;        // [KD][KD] gradient of the state leaving the chunk, transposed likewise
};

__device__ __forceinline__ int64_t row_of(const BW& p, int bb, int t, int h) {
  return (((int64_t)bb * p.L + t) * p.H + h) * KD;
}
// row of an input held at H / hd heads
__device__ __forceinline__ int64_t row_in(const BW& p, int bb, int t, int h, int hd) {
  return (((int64_t)bb * p.L + t) * (p.H / hd) + h / hd) * KD;
}

__device__ __forceinline__ int seg_at(const BW& p, int bb, int t) {
  if (p.seg == nullptr) return 0;
  t = t < p.L ? t : p.L - 1;
  return p.seg[(int64_t)bb * p.L + t];
}

// Per-token document flags of chunk c (threads 0..BC-1).  Segment ids are
// canonical: nondecreasing, and the state entering token 0 belongs to id 0.
__device__ __forceinline__ void chunk_docs(const BW& p, int bb, int t0, int* sseg, int* scar, int* slast) {
  const int t = threadIdx.x;
  const int prev = t0 == 0 ? 0 : seg_at(p, bb, t0 - 1);
  const int s = seg_at(p, bb, t0 + t);
  sseg[t] = s;
  scar[t] = s == prev;
  slast[t] = s == seg_at(p, bb, t0 + BC - 1);
}

// 2^x for x <= 0 (v_exp_f32; results below 2^-126 flush to zero, which no
// gradient here can resolve anyway)
__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(fminf(x, 0.f)); }

__device__ __forceinline__ float4 ld4g(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ float4 zero_f4() { return make_float4(0.f, 0.f, 0.f, 0.f); }
// 4 consecutive elements of f32 or bf16 storage, as f32
__device__ __forceinline__ float4 ld4_dt(const void* p, int64_t i, int dt) {
  if (dt == DT_BF16) {
    const bf16x4 x = *reinterpret_cast<const bf16x4*>((const bf16*)p + i);
    return make_float4((float)x[0], (float)x[1], (float)x[2], (float)x[3]);
  }
  return ld4g((const float*)p + i);
}
__device__ __forceinline__ float f4at(const float4& v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

// 8 values of a 128-wide row at the fragment positions of slab s:
// x[0..3] = row[32s + 4q .. +3], x[4..7] = row[32s + 16 + 4q .. +3]
__device__ __forceinline__ void row8(const float* rowp, int s, int q, float* x) {
  const float4 a = ld4g(rowp + 32 * s + 4 * q);
  const float4 b = ld4g(rowp + 32 * s + 16 + 4 * q);
  x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
  x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}

__device__ __forceinline__ Frag<false> fr8(const float* x) { return make_frag<false>(x); }

// The scan operands Wm, Kc (chunk x 128) and WT, KcT (128 x chunk) are kept
// in the order the scans' fragments read them: a 16-row block and 32-column
// slab is two runs of 64 lanes x 4 floats, lane q * 16 + r holding row r,
// columns 4q..4q+3 of the slab's first (run 0) or second (run 1) 16 columns.
// One fragment load is one contiguous 1 KB run; four consecutive columns
// from a multiple of 4 stay contiguous.  ns = 32-column slabs per row.
__device__ __forceinline__ int gofs(int i, int c, int ns) {
  const int cc = c & 31;
  return ((((i >> 4) * ns + (c >> 5)) * 2 + (cc >> 4)) * 64 + ((cc & 15) >> 2) * 16 + (i & 15)) * 4 + (c & 3);
}
// bf16 mode keeps the four scan operands split: run pair (blk, s) is 64
// lanes x 8 high bf16 words, then 64 lanes x 8 low words, element (i, c) at
// index e = 4 * (run) + (c & 3) of its lane (the same bytes as the fp32
// pair).  op_put4 / op_put8 / op_get8 store and load either form.
__device__ __forceinline__ int bofs(int i, int c, int ns) {
  const int cc = c & 31;
  return ((i >> 4) * ns + (c >> 5)) * 1024 + (((cc & 15) >> 2) * 16 + (i & 15)) * 8 + (cc >> 4) * 4 + (c & 3);
}
// four consecutive columns c..c+3, c a multiple of 4
__device__ __forceinline__ void op_put4(bool bf, float* arr, int i, int c, int ns, float4 v) {
  if (bf) {
    bf16* b = reinterpret_cast<bf16*>(arr) + bofs(i, c, ns);
    const float x[4] = {v.x, v.y, v.z, v.w};
    bf16x4 h, lo;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      h[e] = (bf16)x[e];
      lo[e] = (bf16)(x[e] - (float)h[e]);
    }
    *reinterpret_cast<bf16x4*>(b) = h;
    *reinterpret_cast<bf16x4*>(b + 512) = lo;
  } else {
    *reinterpret_cast<float4*>(arr + gofs(i, c, ns)) = v;
  }
}
// the 8 values of one lane of a run pair: columns c..c+3 and c+16..c+19 of
// row i (c = 32 s + 4 q); neighbouring lanes store neighbouring 16 bytes
__device__ __forceinline__ void op_put8(bool bf, float* arr, int i, int c, int ns, const float* x) {
  if (bf) {
    bf16* b = reinterpret_cast<bf16*>(arr) + bofs(i, c, ns);
    bf16x8 h, lo;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      h[e] = (bf16)x[e];
      lo[e] = (bf16)(x[e] - (float)h[e]);
    }
    *reinterpret_cast<bf16x8*>(b) = h;
    *reinterpret_cast<bf16x8*>(b + 512) = lo;
  } else {
    *reinterpret_cast<float4*>(arr + gofs(i, c, ns)) = make_float4(x[0], x[1], x[2], x[3]);
    *reinterpret_cast<float4*>(arr + gofs(i, c + 16, ns)) = make_float4(x[4], x[5], x[6], x[7]);
  }
}
// the 8 values op_put8 stores for one lane of a run pair
template <bool BF>
__device__ __forceinline__ void op_get8(const float* arr, int i, int c, int ns, float* x) {
  if constexpr (BF) {
    const bf16* b = reinterpret_cast<const bf16*>(arr) + bofs(i, c, ns);
    const bf16x8 h = *reinterpret_cast<const bf16x8*>(b);
    const bf16x8 lo = *reinterpret_cast<const bf16x8*>(b + 512);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = (float)h[e] + (float)lo[e];
  } else {
    const float4 a = ld4g(arr + gofs(i, c, ns)), d = ld4g(arr + gofs(i, c + 16, ns));
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = d.x; x[5] = d.y; x[6] = d.z; x[7] = d.w;
  }
}
// PT (128 x 128) and U0T (128 x chunk) in accumulator order: a 16 x 16 tile
// is one run of 64 lanes x 4 floats, lane q * 16 + r holding row r, columns
// 4q..4q+3.  nt = 16-column tiles per row.
__device__ __forceinline__ int aofs(int r, int c, int nt) {
  return (((r >> 4) * nt + (c >> 4)) * 64 + ((c & 15) >> 2) * 16 + (r & 15)) * 4 + (c & 3);
}
// the 8 fragment values of lane l in run pair (blk, s) of a gofs array
__device__ __forceinline__ void frag_run(const float* arr, int blk, int s, int ns, int l, float* x) {
  const float* b = arr + ((blk * ns + s) * 2) * 256 + 4 * l;
  const float4 a = ld4g(b);
  const float4 c = ld4g(b + 256);
  x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
  x[4] = c.x; x[5] = c.y; x[6] = c.z; x[7] = c.w;
}

// A 16 x 32 product operand from 8 fp32 values in fragment order: fp32 mode
// keeps them (v_mfma_f32_16x16x4_f32), bf16 mode splits them into high and
// low bf16 words (x = hi + lo to 16 significant bits) for the split product
// hi*hi + hi*lo + lo*hi on v_mfma_f32_16x16x32_bf16.
template <bool BF> struct Op;
template <> struct Op<false> {
  using F = Frag<false>;
  static __device__ __forceinline__ F make(const float* x) { return make_frag<false>(x); }
  static __device__ __forceinline__ void mac(f32x4& acc, const F& a, const F& b) { mma(acc, a, b); }
};
template <> struct Op<true> {
  using F = Pol<true>::F3;
  static __device__ __forceinline__ F make(const float* x) { return Pol<true>::f3(x); }
  static __device__ __forceinline__ void mac(f32x4& acc, const F& a, const F& b) { Pol<true>::m33(acc, a, b); }
};

// ---------------------------------------------------------------------------
// k_bw_intra
// ---------------------------------------------------------------------------
template <bool BF>
__global__ __launch_bounds__(NT) void k_bw_intra(BW p) {
  using O = Op<BF>;
  __shared__ float sG[BC][KP];
  __shared__ float sA[BC][CP];   // A, then T
  __shared__ float sM[BC][CP];
  __shared__ float sW[BC][KP];    // b * k of the chunk, then W
  __shared__ float sQ[BC][KP];    // q of the chunk
  __shared__ float sTot[4][KD];   // per-quarter decay totals of the scan
  __shared__ float sX[16][17];    // one 16 x 16 block in transit (T substitution)
  __shared__ int sseg[BC], scar[BC], slast[BC];
  __shared__ int sSafe[NWV];
  __shared__ uint64_t sStarts;   // bit i: a document starts at token i (i > 0)

  const int tid = threadIdx.x, l = tid & 63, wv = tid >> 6, q = l >> 4, l16 = l & 15;
  // Persistent: workgroup blockIdx.x takes units blockIdx.x, + gridDim.x, ...
  // and loads the next unit's k and g (a thread's 4 tokens x 4 channels)
  // during the current one's last phase, so only its first unit waits on
  // them; q and b are loaded at the unit's start and staged after Kc.
  constexpr int SIT = BC * KD / 4 / NT;
  static_assert(SIT == 4 && NT == 16 * (KD / 4) && BC == 64, "token mapping of the staging loop");
  const int nu = p.B * p.H * p.NC;
  float4 nk[SIT], ng[SIT];
  auto stage_load = [&](int un) {
    const int c = un % p.NC, bh = un / p.NC, h = bh % p.H, bb = bh / p.H;
    const int t0 = (p.c0 + c) * BC;
#pragma unroll
    for (int it = 0; it < SIT; ++it) {
      const int c4 = tid % (KD / 4), i = 4 * (tid / (KD / 4)) + it;
      nk[it] = ng[it] = zero_f4();
      if (t0 + i < p.L) {
        nk[it] = ld4g(p.k + row_in(p, bb, t0 + i, h, p.qk_hd) + 4 * c4);
        ng[it] = ld4g(p.g + row_in(p, bb, t0 + i, h, p.gb_hd) + 4 * c4);
      }
    }
  };
  if (blockIdx.x < (unsigned)nu) stage_load(blockIdx.x);
  for (int u = blockIdx.x; u < nu; u += gridDim.x) {
  const int c = u % p.NC, bh = u / p.NC, h = bh % p.H, bb = bh / p.H;
  const int t0 = (p.c0 + c) * BC;
  float* G = p.G + (int64_t)u * CK;

  if (tid < BC) {   // wave 0
    chunk_docs(p, bb, t0, sseg, scar, slast);
    const int sg = sseg[tid];
    const int sp = __shfl_up(sg, 1);   // every lane takes part (lane 0 gets its own value)
    const uint64_t st = __ballot(tid > 0 && sg != sp);
    if (tid == 0) sStarts = st;
  }
  // stage the log2-decay (rows past the sequence end are zero); k stays in
  // registers for Kc and beta = b k; q and b arrive during the decay scan
  float4 kst[SIT], qst[SIT], bst[SIT];
#pragma unroll
  for (int it = 0; it < SIT; ++it) {
    // a thread holds 4 consecutive tokens x 4 channels
    const int c4 = tid % (KD / 4), i = 4 * (tid / (KD / 4)) + it;
    const float4 gv = ng[it];
    kst[it] = nk[it];
    *reinterpret_cast<float4*>(&sG[i][4 * c4]) =
        make_float4(gv.x * kLog2e, gv.y * kLog2e, gv.z * kLog2e, gv.w * kLog2e);
    qst[it] = bst[it] = zero_f4();
    if (t0 + i < p.L) {
      qst[it] = ld4g(p.q + row_in(p, bb, t0 + i, h, p.qk_hd) + 4 * c4);
      bst[it] = ld4g(p.b + row_in(p, bb, t0 + i, h, p.gb_hd) + 4 * c4);
    }
  }
  lds_barrier();
  // ---- cumulative decay (log2 units): channel tid % 128, quarter tid / 128 --
  // The sum restarts at every document start inside the chunk.  Only pairs of
  // one document use a difference G_i - G_j, and the chunk-start terms
  // (carry, lam) only tokens of the chunk's first document, so every use is
  // unchanged; but a later document's small decays are no longer added to
  // an earlier document's large sum, where fp32 would absorb them
  // (reference gdn2.py mask_lambda_by_doc, tests/test_precision_flags.py).
  {
    const int ch = tid & (KD - 1), qt = tid >> 7;
    // wave-uniform (scalar registers): the chunk's starts, this quarter's
    const uint64_t stm = sStarts;
    const uint32_t slo = __builtin_amdgcn_readfirstlane((uint32_t)stm);
    const uint32_t shi = __builtin_amdgcn_readfirstlane((uint32_t)(stm >> 32));
    const uint32_t qm = ((qt < 2 ? slo : shi) >> (16 * (qt & 1))) & 0xffffu;
    const int first = qm ? __builtin_ctz(qm) : BC / 4;   // BC / 4: none
    float part[BC / 4];
    float acc = 0.f;
#pragma unroll
    for (int t = 0; t < BC / 4; ++t) {
      if ((qm >> t) & 1u) acc = 0.f;
      acc += sG[16 * qt + t][ch];
      part[t] = acc;
    }
    sTot[qt][ch] = acc;   // the sum since the quarter's last start (or its whole sum)
    lds_barrier();
    float off = 0.f;
#pragma unroll
    for (int s2 = 0; s2 < 3; ++s2) {
      if (s2 < qt) off = ((((s2 < 2 ? slo : shi) >> (16 * (s2 & 1))) & 0xffffu) ? 0.f : off) + sTot[s2][ch];
    }
#pragma unroll
    for (int t = 0; t < BC / 4; ++t) sG[16 * qt + t][ch] = part[t] + (t < first ? off : 0.f);
  }
  lds_barrier();
  // G (coalesced), lam, Kc from the staged k into LDS (channels 0..63 in sA,
  // 64..127 in sM: both are free until A and M), and per 16-token block
  // whether its decay span allows the factored (MFMA) diagonal tiles
  {
#pragma unroll
    for (int it = 0; it < SIT; ++it) {
      const int c4 = tid % (KD / 4), i = 4 * (tid / (KD / 4)) + it;
      const float4 gi = *reinterpret_cast<const float4*>(&sG[i][4 * c4]);
      const float4 gl = *reinterpret_cast<const float4*>(&sG[BC - 1][4 * c4]);
      *reinterpret_cast<float4*>(G + i * KD + 4 * c4) = gi;
      const bool ok = slast[i] && t0 + i < p.L;
      const float4 k4 = kst[it];
      const float4 kc = ok ? make_float4(k4.x * ex2(gl.x - gi.x), k4.y * ex2(gl.y - gi.y),
                                         k4.z * ex2(gl.z - gi.z), k4.w * ex2(gl.w - gi.w))
                           : zero_f4();
      *reinterpret_cast<float4*>(c4 < KD / 8 ? &sA[i][4 * c4] : &sM[i][4 * c4 - KD / 2]) = kc;
    }
    if (tid < KD) p.lam[(int64_t)u * KD + tid] = scar[BC - 1] ? ex2(sG[BC - 1][tid]) : 0.f;
    // block tid / 128 spans 2^{G_m - G_{m+15}} <= 2^64 in channel tid % 128,
    // and no document starts after its first row (G is monotone in it)
    const int ch = tid & (KD - 1), blk = tid >> 7;
    const float span = sG[16 * blk][ch] - sG[16 * blk + 15][ch];
    const bool one_doc = sseg[16 * blk] == sseg[16 * blk + 15];   // ids are nondecreasing
    const bool safe = one_doc && __all(span <= 64.f);
    if (l == 0) sSafe[wv] = safe;
  }
  // q and beta = b k
#pragma unroll
  for (int it = 0; it < SIT; ++it) {
    const int c4 = tid % (KD / 4), i = 4 * (tid / (KD / 4)) + it;
    const float4 k4 = kst[it], b4 = bst[it];
    *reinterpret_cast<float4*>(&sQ[i][4 * c4]) = qst[it];
    *reinterpret_cast<float4*>(&sW[i][4 * c4]) = make_float4(b4.x * k4.x, b4.y * k4.y, b4.z * k4.z, b4.w * k4.w);
  }
  lds_barrier();
  // Kc and Kc^T in the scan operand order: per task one lane's run pair
  {
    float* Kc = p.Kc + (int64_t)u * CK;
    float* KcT = p.KcT + (int64_t)u * CK;
    auto kc_at = [&](int i, int ch) { return ch < KD / 2 ? sA[i][ch] : sM[i][ch - KD / 2]; };
    for (int task = tid; task < BC * KD / 8; task += NT) {
      const int ln = task & 63, pr = task >> 6;
      float x[8];
      {
        const int blk = pr / (KD / 32), s = pr % (KD / 32);
        const int i = 16 * blk + (ln & 15), cc = 32 * s + 4 * (ln >> 4);
        const float* rp = cc < KD / 2 ? &sA[i][cc] : &sM[i][cc - KD / 2];
        const float4 x0 = *reinterpret_cast<const float4*>(rp);
        const float4 x1 = *reinterpret_cast<const float4*>(rp + 16);
        x[0] = x0.x; x[1] = x0.y; x[2] = x0.z; x[3] = x0.w; x[4] = x1.x; x[5] = x1.y; x[6] = x1.z; x[7] = x1.w;
        op_put8(p.bf, Kc, i, cc, KD / 32, x);
      }
      {
        const int blk = pr / (BC / 32), s = pr % (BC / 32);
        const int ch = 16 * blk + (ln & 15), tc = 32 * s + 4 * (ln >> 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x[e] = kc_at(tc + e, ch);
          x[4 + e] = kc_at(tc + 16 + e, ch);
        }
        op_put8(p.bf, KcT, ch, tc, BC / 32, x);
      }
    }
  }
  lds_barrier();
  // A and M write their lower-triangle 16 x 16 tiles whole; the six tiles
  // above the diagonal stay zero
  for (int idx = tid; idx < 6 * 256; idx += NT) {
    const int t = idx >> 8, e = idx & 255;
    const int I = t < 3 ? 0 : (t < 5 ? 1 : 2), J = t < 3 ? t + 1 : (t < 5 ? t - 1 : 3);
    sA[16 * I + (e >> 4)][16 * J + (e & 15)] = 0.f;
    sM[16 * I + (e >> 4)][16 * J + (e & 15)] = 0.f;
  }

  // ---- A (strict) and M (with diagonal), 16x16 tiles of the lower triangle --
  // A pair (i, j) with j <= m <= i is formed as (x_i e^{G_i - G_m}) (k_j e^{G_m - G_j}),
  // m = the first row of i's block.  Off the diagonal both factors are <= 1;
  // on the diagonal the column factor is >= 1, which is used only where the
  // block's decay span keeps it below 2^64 -- otherwise every element takes
  // e^{G_i - G_j} directly.
  // one task per lower-triangle tile (I, J) forms both A_IJ and M_IJ: they
  // share the column operand k_j e^{G_m - G_j} and the row factor
  // e^{G_i - G_m}
  for (int tt = wv; tt < 10; tt += NWV) {
    const int I = (tt >= 1) + (tt >= 3) + (tt >= 6);
    const int J = tt - I * (I + 1) / 2;
    const bool diag = J == I;
    float resA[4], resM[4];
    if (!diag || (sSafe[2 * I] & sSafe[2 * I + 1])) {
      const int m = 16 * I;
      const int i = 16 * I + l16, j = 16 * J + l16;
      const bool vi = t0 + i < p.L, vj = t0 + j < p.L;
      const float* kj = p.k + row_in(p, bb, vj ? t0 + j : 0, h, p.qk_hd);
      f32x4 accA = zero4(), accM = zero4();
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        float xa[8], xq[8], xb[8], gi[8], gm[8], gj[8];
        row8(&sW[i][0], s, q, xa);
        row8(&sQ[i][0], s, q, xq);
        row8(kj, s, q, xb);
        row8(&sG[i][0], s, q, gi);
        row8(&sG[m][0], s, q, gm);
        row8(&sG[j][0], s, q, gj);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float fi = vi ? ex2(gi[e] - gm[e]) : 0.f;
          xa[e] *= fi;
          xq[e] *= fi;
          const float fb = diag ? __builtin_amdgcn_exp2f(gm[e] - gj[e]) : ex2(gm[e] - gj[e]);
          xb[e] = vj ? xb[e] * fb : 0.f;
        }
        const Frag<false> fbk = fr8(xb);
        mma(accA, fr8(xa), fbk);
        mma(accM, fr8(xq), fbk);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        resA[e] = accA[e];
        resM[e] = accM[e];
      }
    } else {
      // diagonal block with a large decay span: e^{G_i - G_j} per element
      const int j = 16 * I + l16;
      const bool vj = t0 + j < p.L;
      const float* kj = p.k + row_in(p, bb, vj ? t0 + j : 0, h, p.qk_hd);
#pragma unroll
      for (int e = 0; e < 4; ++e) resA[e] = resM[e] = 0.f;
#pragma unroll 8
      for (int r4 = 0; r4 < KD / 4; ++r4) {
        const float4 kv = ld4g(kj + 4 * r4);
        const float4 gjv = *reinterpret_cast<const float4*>(&sG[j][4 * r4]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 16 * I + 4 * q + e;
          const float4 wv4 = *reinterpret_cast<const float4*>(&sW[i][4 * r4]);
          const float4 qv4 = *reinterpret_cast<const float4*>(&sQ[i][4 * r4]);
          const float4 giv = *reinterpret_cast<const float4*>(&sG[i][4 * r4]);
          const float f0 = kv.x * ex2(giv.x - gjv.x), f1 = kv.y * ex2(giv.y - gjv.y);
          const float f2 = kv.z * ex2(giv.z - gjv.z), f3 = kv.w * ex2(giv.w - gjv.w);
          resA[e] += wv4.x * f0 + wv4.y * f1 + wv4.z * f2 + wv4.w * f3;
          resM[e] += qv4.x * f0 + qv4.y * f1 + qv4.z * f2 + qv4.w * f3;
        }
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 16 * I + 4 * q + e, j = 16 * J + l16;
      const bool same = sseg[i] == sseg[j] && t0 + i < p.L && t0 + j < p.L;
      sA[i][j] = same && j < i ? resA[e] : 0.f;
      sM[i][j] = same && j <= i ? resM[e] : 0.f;
    }
  }
  // w and v of this lane's W / U0 operands, loaded now and used after T
  static_assert(TPW == 1, "one 16-column tile per wave");
  float wvw[2][8], wvv[2][8];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int j = 32 * s + pi_k(q, e), r = 16 * wv + l16;
      const bool vj = t0 + j < p.L;
      const int64_t ro = row_of(p, bb, vj ? t0 + j : 0, h) + r;
      wvw[s][e] = vj ? p.w[ro] : 0.f;
      wvv[s][e] = vj ? ld_f(p.v, ro, p.v_dt) : 0.f;
    }
  lds_barrier();

  // ---- T = (I + A)^-1, blocked, by wave 0 ----------------------------------
  // The four 16x16 diagonal blocks D_I = (I + A_II)^-1 by forward substitution
  // (lane = block I, column c); then block rows I = 1..3 in order,
  // T_IJ = -D_I sum_{K=J}^{I-1} A_IK T_KJ on v_mfma_f32_16x16x4f32.  Each T
  // block overwrites the A block it replaces once no later product needs it.
  if (wv == 0) {
    {
      const int I = l >> 4, cc = l & 15;
      float t[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float acc = r == cc ? 1.f : 0.f;
#pragma unroll
        for (int s2 = 0; s2 < r; ++s2) acc -= sA[16 * I + r][16 * I + s2] * t[s2];
        t[r] = acc;
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) sA[16 * I + r][16 * I + cc] = t[r];
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
    for (int I = 1; I < 4; ++I) {
#pragma unroll
      for (int J = 0; J < I; ++J) {
        f32x4 x = zero4();
#pragma unroll
        for (int K = J; K < I; ++K)
#pragma unroll
          for (int kk = 0; kk < 4; ++kk)
            x = __builtin_amdgcn_mfma_f32_16x16x4f32(sA[16 * I + l16][16 * K + 4 * kk + q],
                                                      sA[16 * K + 4 * kk + q][16 * J + l16], x, 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) sX[4 * q + e][l16] = x[e];
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        f32x4 y = zero4();
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
          y = __builtin_amdgcn_mfma_f32_16x16x4f32(sA[16 * I + l16][16 * I + 4 * kk + q], sX[4 * kk + q][l16], y,
                                                    0, 0, 0);
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
        for (int e = 0; e < 4; ++e) sA[16 * I + 4 * q + e][16 * J + l16] = -y[e];
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
      }
    }
    float* TT = p.TT + (int64_t)u * CC + l * BC;
#pragma unroll
    for (int i4 = 0; i4 < BC / 4; ++i4)
      *reinterpret_cast<float4*>(TT + 4 * i4) =
          make_float4(sA[4 * i4][l], sA[4 * i4 + 1][l], sA[4 * i4 + 2][l], sA[4 * i4 + 3][l]);
  } else {
    const int t2 = tid - 64;
    float* MT = p.MT + (int64_t)u * CC;
    for (int idx = t2; idx < CC; idx += NT - 64) {
      const int j = idx / BC, i = idx % BC;
      MT[idx] = sM[i][j];
    }
  }
  lds_barrier();
  // bf16 mode: T (final, and already written out as T^T) is stored over itself
  // as high / low bf16 planes, split once for every wave's W / U0 products
  if constexpr (BF) {
    float tv[CC / NT];
#pragma unroll
    for (int e = 0; e < CC / NT; ++e) {
      const int idx = tid + NT * e;
      tv[e] = sA[idx / BC][idx % BC];
    }
    lds_barrier();
    bf16 (*th)[CP] = reinterpret_cast<bf16 (*)[CP]>(&sA[0][0]);
#pragma unroll
    for (int e = 0; e < CC / NT; ++e) {
      const int idx = tid + NT * e;
      const bf16 h = (bf16)tv[e];
      th[idx / BC][idx % BC] = h;
      th[BC + idx / BC][idx % BC] = (bf16)(tv[e] - (float)h);
    }
    lds_barrier();
  }

  // ---- W = T diag(carry) (b k e^G), U0 = T (w v) ---------------------------
  {
    f32x4 aw[4][TPW], au[4][TPW];
#pragma unroll
    for (int I = 0; I < 4; ++I)
#pragma unroll
      for (int R2 = 0; R2 < TPW; ++R2) { aw[I][R2] = zero4(); au[I][R2] = zero4(); }
    static_assert(TPW == 1, "one 16-column tile per wave");
    const int r = 16 * wv + l16;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      // this lane's b k e^G and w v column fragments, then each row block's
      // T fragment just before its two products (one T fragment live at a time)
      float xb[8], xu[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int j = 32 * s + pi_k(q, e);
        xb[e] = scar[j] ? sW[j][r] * ex2(sG[j][r]) : 0.f;
        xu[e] = wvw[s][e] * wvv[s][e];
      }
      const typename O::F fb = O::make(xb), fu = O::make(xu);
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        if (s == 1 && I < 2) continue;   // T is lower triangular: rows < 32 x columns >= 32 are zero
        typename O::F a;
        if constexpr (BF) {
          const bf16 (*th)[CP] = reinterpret_cast<const bf16 (*)[CP]>(&sA[0][0]);
          const int rr = 16 * I + l16;
          const bf16x4 h0 = *reinterpret_cast<const bf16x4*>(&th[rr][32 * s + 4 * q]);
          const bf16x4 h1 = *reinterpret_cast<const bf16x4*>(&th[rr][32 * s + 16 + 4 * q]);
          const bf16x4 l0 = *reinterpret_cast<const bf16x4*>(&th[BC + rr][32 * s + 4 * q]);
          const bf16x4 l1 = *reinterpret_cast<const bf16x4*>(&th[BC + rr][32 * s + 16 + 4 * q]);
          a.hi.v = bf16x8{h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
          a.lo.v = bf16x8{l0[0], l0[1], l0[2], l0[3], l1[0], l1[1], l1[2], l1[3]};
        } else {
          float x[8];
          const float* rp = &sA[16 * I + l16][32 * s];
          const float4 x0 = *reinterpret_cast<const float4*>(rp + 4 * q);
          const float4 x1 = *reinterpret_cast<const float4*>(rp + 16 + 4 * q);
          x[0] = x0.x; x[1] = x0.y; x[2] = x0.z; x[3] = x0.w; x[4] = x1.x; x[5] = x1.y; x[6] = x1.z; x[7] = x1.w;
          a = fr8(x);
        }
        O::mac(aw[I][0], a, fb);
        O::mac(au[I][0], a, fu);
      }
    }
    float* WT = p.WT + (int64_t)u * CK;
    float* U0T = p.U0T + (int64_t)u * CK;
    lds_barrier();   // every wave has read b k from sW
#pragma unroll
    for (int I = 0; I < 4; ++I)
#pragma unroll
      for (int R2 = 0; R2 < TPW; ++R2) {
        const int r = 16 * (TPW * wv + R2) + l16;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 16 * I + 4 * q + e;
          sW[i][r] = aw[I][R2][e];
        }
        *reinterpret_cast<float4*>(U0T + aofs(r, 16 * I + 4 * q, BC / 16)) =
            make_float4(au[I][R2][0], au[I][R2][1], au[I][R2][2], au[I][R2][3]);
        op_put4(p.bf, WT, r, 16 * I + 4 * q, BC / 32, make_float4(aw[I][R2][0], aw[I][R2][1], aw[I][R2][2], aw[I][R2][3]));
      }
  }
  lds_barrier();
  // the chunk's dO (rows past the sequence end zero), loaded here for the P^T
  // phase at the end (not earlier: it would hold 16 registers through W / U0)
  float4 dov[BC * KD / 4 / NT];
#pragma unroll
  for (int it = 0; it < BC * KD / 4 / NT; ++it) {
    const int idx = tid + NT * it, i = idx / (KD / 4), c4 = idx % (KD / 4);
    dov[it] = t0 + i < p.L ? ld4_dt(p.dout, row_of(p, bb, t0 + i, h) + 4 * c4, p.dout_dt) : zero_f4();
  }
  // W in the scan operand order from sW: per task one lane's run pair (rows
  // of 16-row block blk, slab s)
  {
    float* Wm = p.Wm + (int64_t)u * CK;
    for (int task = tid; task < BC * KD / 8; task += NT) {
      const int ln = task & 63, pr = task >> 6, blk = pr / (KD / 32), s = pr % (KD / 32);
      const int i = 16 * blk + (ln & 15), cc = 32 * s + 4 * (ln >> 4);
      const float4 x0 = *reinterpret_cast<const float4*>(&sW[i][cc]);
      const float4 x1 = *reinterpret_cast<const float4*>(&sW[i][cc + 16]);
      const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
      op_put8(p.bf, Wm, i, cc, KD / 32, x);
    }
  }

  if (u + (int)gridDim.x < nu) stage_load(u + gridDim.x);   // the next unit's inputs

  // ---- Xf = diag(carry) q e^G - M W, then P^T = (Xf^T dO)^T ------------------
  {
    f32x4 ax[4][TPW];
#pragma unroll
    for (int I = 0; I < 4; ++I)
#pragma unroll
      for (int R2 = 0; R2 < TPW; ++R2) ax[I][R2] = zero4();
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      // this lane's W column fragment, then each row block's M fragment just
      // before its product
      float xb[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) xb[e] = sW[32 * s + pi_k(q, e)][16 * wv + l16];
      const typename O::F fb = O::make(xb);
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        if (s == 1 && I < 2) continue;   // M is lower triangular
        float x[8];
        const float* rp = &sM[16 * I + l16][32 * s];
        const float4 x0 = *reinterpret_cast<const float4*>(rp + 4 * q);
        const float4 x1 = *reinterpret_cast<const float4*>(rp + 16 + 4 * q);
        x[0] = x0.x; x[1] = x0.y; x[2] = x0.z; x[3] = x0.w; x[4] = x1.x; x[5] = x1.y; x[6] = x1.z; x[7] = x1.w;
        O::mac(ax[I][0], O::make(x), fb);
      }
    }
    float xf[4][4];
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      const int r = 16 * wv + l16;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = 16 * I + 4 * q + e;
        const float qe = scar[i] ? sQ[i][r] * ex2(sG[i][r]) : 0.f;
        xf[I][e] = qe - ax[I][0][e];
      }
    }
    // Xf replaces W in sW and dO replaces q in sQ once every wave is done with them
    lds_barrier();
#pragma unroll
    for (int I = 0; I < 4; ++I)
#pragma unroll
      for (int e = 0; e < 4; ++e) sW[16 * I + 4 * q + e][16 * wv + l16] = xf[I][e];
#pragma unroll
    for (int it = 0; it < BC * KD / 4 / NT; ++it) {
      const int idx = tid + NT * it, i = idx / (KD / 4), c4 = idx % (KD / 4);
      *reinterpret_cast<float4*>(&sQ[i][4 * c4]) = dov[it];
    }
    lds_barrier();
    // P^T rows v = 16 w .. 16 w + 15, all 128 k: P[k][v] = sum_i Xf[i][k] dO[i][v]
    // is the state-free term of the reverse scan's step
    typename O::F fdo[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      float xb[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) xb[e] = sQ[32 * s + pi_k(q, e)][16 * wv + l16];
      fdo[s] = O::make(xb);
    }
    float* PT = p.PT + (int64_t)u * KK;
#pragma unroll
    for (int kt = 0; kt < KD / 16; ++kt) {
      f32x4 acc = zero4();
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        float xa[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) xa[e] = sW[32 * s + pi_k(q, e)][16 * kt + l16];
        O::mac(acc, O::make(xa), fdo[s]);
      }
      *reinterpret_cast<float4*>(PT + aofs(16 * wv + l16, 16 * kt + 4 * q, KD / 16)) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    }
  }
  lds_barrier();   // the next unit reuses the LDS
  }
}

// ---------------------------------------------------------------------------
// chain_run: one (batch, head, block of 16 CT state columns) per workgroup;
// wave w owns state rows 32w..32w+31 of the CT column tiles, so every operand
// fragment it loads serves CT tiles.  The 128 x 16 CT state block lives in
// LDS in fragment order ([tile][slab][lane][8]).
//   forward  (BWD = false):  Y = U0 - W S ;  S <- lam * S + Kc^T Y
//   backward (BWD = true):   Z = -Kc dS  ;  dS <- lam * dS + Xf^T dO + W^T Z
// Every operand but the state is known before the scan, so each step loads
// the next chunk's operands while it computes.  The loads bound the step:
// the operand rows are the same for every column block of a head, so wider
// blocks (CT = 2 in bf16 mode, where the split-bf16 products keep the MFMA
// time per step small) divide the bytes per column.  bf16 mode reads the
// operands split (k_bw_intra stores them so) and keeps the state in LDS split.
// ---------------------------------------------------------------------------
template <bool BF> constexpr int chain_tiles() { return BF ? 2 : 1; }

template <bool BF>
struct ChainOps {
  static constexpr int CT = chain_tiles<BF>();
  typename Op<BF>::F a[4];      // W (forward) / Kc (backward): this wave's 16 tokens, 4 slabs
  typename Op<BF>::F b[2][2];   // Kc^T (forward) / W^T (backward): this wave's 32 state rows, 2 slabs
  float4 pp[CT][2];             // (Xf^T dO) entries of this lane's state rows (backward)
  float4 u[CT];                 // U0 tile entries of this lane (forward)
  float4 lm[2];                 // lam of this lane's state rows
};

// run pair (blk, s) of an operand array as an MFMA fragment of lane l
template <bool BF>
__device__ __forceinline__ typename Op<BF>::F op_frag(const float* arr, int blk, int s, int ns, int l) {
  if constexpr (BF) {
    const bf16* b = reinterpret_cast<const bf16*>(arr) + (blk * ns + s) * 1024 + 8 * l;
    typename Op<true>::F f;
    f.hi.v = *reinterpret_cast<const bf16x8*>(b);
    f.lo.v = *reinterpret_cast<const bf16x8*>(b + 512);
    return f;
  } else {
    float x[8];
    frag_run(arr, blk, s, ns, l, x);
    return fr8(x);
  }
}

template <bool BWD, bool BF>
__device__ __forceinline__ void chain_load(const BW& p, int bh, int c, int col0, int wv, int l, ChainOps<BF>& o) {
  constexpr int CT = ChainOps<BF>::CT;
  const int q = l >> 4, l16 = l & 15;
  const int64_t u = (int64_t)bh * p.NC + c;
  const float* Aarr = (BWD ? p.Kc : p.Wm) + u * CK;
  const float* Barr = (BWD ? p.WT : p.KcT) + u * CK;
#pragma unroll
  for (int s = 0; s < 4; ++s) o.a[s] = op_frag<BF>(Aarr, wv, s, KD / 32, l);
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) o.b[tt][s2] = op_frag<BF>(Barr, 2 * wv + tt, s2, BC / 32, l);
#pragma unroll
    for (int j = 0; j < CT; ++j)
      if (BWD) o.pp[j][tt] = ld4g(p.PT + u * KK + aofs(col0 + 16 * j + l16, 32 * wv + 16 * tt + 4 * q, KD / 16));
    o.lm[tt] = ld4g(p.lam + u * KD + 32 * wv + 16 * tt + 4 * q);
  }
#pragma unroll
  for (int j = 0; j < CT; ++j)
    if (!BWD) o.u[j] = ld4g(p.U0T + u * CK + aofs(col0 + 16 * j + l16, 16 * wv + 4 * q, BC / 16));
}

// LDS copy of the state (S) and of the Y / Z tile, in fragment order; split
// into bf16 words in bf16 mode
template <bool BF, int CT> struct ChainLds;
template <int CT> struct ChainLds<false, CT> {
  float S[CT][4][64][8];
  float Y[CT][2][64][8];
  __device__ __forceinline__ void put_s(int j, int wv, int l, const f32x4& s0, const f32x4& s1) {
    *reinterpret_cast<float4*>(&S[j][wv][l][0]) = make_float4(s0[0], s0[1], s0[2], s0[3]);
    *reinterpret_cast<float4*>(&S[j][wv][l][4]) = make_float4(s1[0], s1[1], s1[2], s1[3]);
  }
  __device__ __forceinline__ void put_y(int j, int wv, int l, const f32x4& y) {
    *reinterpret_cast<float4*>(&Y[j][wv >> 1][l][4 * (wv & 1)]) = make_float4(y[0], y[1], y[2], y[3]);
  }
  __device__ __forceinline__ Frag<false> s_frag(int j, int s, int l) const { return fr8(&S[j][s][l][0]); }
  __device__ __forceinline__ Frag<false> y_frag(int j, int s, int l) const { return fr8(&Y[j][s][l][0]); }
};
template <int CT> struct ChainLds<true, CT> {
  bf16x8 S[2][CT][4][64];   // [hi, lo]
  bf16x4 Y[2][CT][2][64][2];
  __device__ __forceinline__ void put_s(int j, int wv, int l, const f32x4& s0, const f32x4& s1) {
    bf16x8 h, lo;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = e < 4 ? s0[e] : s1[e - 4];
      h[e] = (bf16)x;
      lo[e] = (bf16)(x - (float)h[e]);
    }
    S[0][j][wv][l] = h;
    S[1][j][wv][l] = lo;
  }
  __device__ __forceinline__ void put_y(int j, int wv, int l, const f32x4& y) {
    bf16x4 h, lo;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      h[e] = (bf16)y[e];
      lo[e] = (bf16)(y[e] - (float)h[e]);
    }
    Y[0][j][wv >> 1][l][wv & 1] = h;
    Y[1][j][wv >> 1][l][wv & 1] = lo;
  }
  __device__ __forceinline__ Pol<true>::F3 s_frag(int j, int s, int l) const {
    Pol<true>::F3 f;
    f.hi.v = S[0][j][s][l];
    f.lo.v = S[1][j][s][l];
    return f;
  }
  __device__ __forceinline__ Pol<true>::F3 y_frag(int j, int s, int l) const {
    Pol<true>::F3 f;
    const bf16x4 h0 = Y[0][j][s][l][0], h1 = Y[0][j][s][l][1], l0 = Y[1][j][s][l][0], l1 = Y[1][j][s][l][1];
    f.hi.v = bf16x8{h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
    f.lo.v = bf16x8{l0[0], l0[1], l0[2], l0[3], l1[0], l1[1], l1[2], l1[3]};
    return f;
  }
};

// one scan over chain x = (batch * H + head) * (8 / CT) + column block
template <bool BWD, bool BF>
__device__ __forceinline__ void chain_run(const BW& p, int x) {
  using O = Op<BF>;
  constexpr int CT = chain_tiles<BF>();
  constexpr int NB = KD / (16 * CT);
  __shared__ ChainLds<BF, CT> sm;
  const int cb = x % NB, bh = x / NB;
  const int col0 = 16 * CT * cb;
  const int tid = threadIdx.x, l = tid & 63, wv = tid >> 6, q = l >> 4, l16 = l & 15;

  f32x4 st[CT][2];
  const float* src = BWD ? p.dfin : p.init;
#pragma unroll
  for (int j = 0; j < CT; ++j)
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 32 * wv + 16 * tt + 4 * q + e;
        st[j][tt][e] = src ? src[((int64_t)bh * KD + r) * KD + col0 + 16 * j + l16] : 0.f;
      }
#pragma unroll
  for (int j = 0; j < CT; ++j) sm.put_s(j, wv, l, st[j][0], st[j][1]);

  // one scan step on chunk c with operands `o` in registers
  auto step = [&](int c, const ChainOps<BF>& o) {
    const int64_t u = (int64_t)bh * p.NC + c;
    lds_barrier();
    {
      float* X = (BWD ? p.dS : p.S) + u * KK;   // transposed: 4 consecutive k per lane
#pragma unroll
      for (int j = 0; j < CT; ++j)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          const int r0 = 32 * wv + 16 * tt + 4 * q;
          *reinterpret_cast<float4*>(X + (col0 + 16 * j + l16) * KD + r0) =
              make_float4(st[j][tt][0], st[j][tt][1], st[j][tt][2], st[j][tt][3]);
        }
    }
    // Y (or Z) tiles: token rows 16w..16w+15; with one tile, two accumulators
    // halve the dependent MFMA chain on the sequential path
    f32x4 y[CT], y2[CT];
#pragma unroll
    for (int j = 0; j < CT; ++j) y[j] = y2[j] = zero4();
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int j = 0; j < CT; ++j) {
        O::mac(y[j], o.a[s], sm.s_frag(j, s, l));
        O::mac(y2[j], o.a[s + 2], sm.s_frag(j, s + 2, l));
      }
#pragma unroll
    for (int j = 0; j < CT; ++j) {
#pragma unroll
      for (int e = 0; e < 4; ++e) y[j][e] = BWD ? -(y[j][e] + y2[j][e]) : f4at(o.u[j], e) - (y[j][e] + y2[j][e]);
      sm.put_y(j, wv, l, y[j]);
    }
    lds_barrier();
    f32x4 acc[CT][2];
#pragma unroll
    for (int j = 0; j < CT; ++j)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[j][tt][e] = f4at(o.lm[tt], e) * st[j][tt][e];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int j = 0; j < CT; ++j) {
        const auto fy = sm.y_frag(j, s2, l);
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) O::mac(acc[j][tt], o.b[tt][s2], fy);
      }
#pragma unroll
    for (int j = 0; j < CT; ++j) {
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int e = 0; e < 4; ++e) st[j][tt][e] = acc[j][tt][e] + (BWD ? f4at(o.pp[j][tt], e) : 0.f);
      sm.put_s(j, wv, l, st[j][0], st[j][1]);
    }
  };
  // chunk visited at scan position it (clamped: the load past the end is unused)
  auto chunk_at = [&](int it) {
    const int itc = it < p.NC ? it : p.NC - 1;
    return BWD ? p.NC - 1 - itc : itc;
  };
  // two operand sets, alternated (no register copies between steps)
  ChainOps<BF> o0, o1;
  chain_load<BWD>(p, bh, chunk_at(0), col0, wv, l, o0);
  int it = 0;
  for (; it + 1 < p.NC; it += 2) {
    chain_load<BWD>(p, bh, chunk_at(it + 1), col0, wv, l, o1);
    step(chunk_at(it), o0);
    chain_load<BWD>(p, bh, chunk_at(it + 2), col0, wv, l, o0);
    step(chunk_at(it + 1), o1);
  }
  if (it < p.NC) step(chunk_at(it), o0);
  float* dst = BWD ? p.dinit : p.sfin;
  if (dst != nullptr) {
#pragma unroll
    for (int j = 0; j < CT; ++j)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 32 * wv + 16 * tt + 4 * q + e;
          dst[((int64_t)bh * KD + r) * KD + col0 + 16 * j + l16] = st[j][tt][e];
        }
  }
}

// Chains per direction of a launch (B * H heads, 8 / CT column blocks each).
__host__ __device__ constexpr int chains_per_head(bool bf) { return KD / (16 * (bf ? 2 : 1)); }

// Both scans in one launch: they are independent (both read only
// k_bw_intra's products) and each waits mostly on its next chunk's operands.
// nb chains (forward ones first, then the reverse ones when nb = 2 C) over a
// grid of 8 * per blocks: block b runs chain (b % 8) * per + b / 8, so
// consecutive chains -- the column blocks of one head, which read the same
// operand rows -- run on one XCD and share its L2; blocks past nb return at
// once.  C = chains per direction.
template <bool BF>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_bw_chains(BW p, int C, int nb) {
  const int per = gridDim.x >> 3;
  const int x = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
  if (x >= nb) return;
  if (x < C) chain_run<false, BF>(p, x);
  else chain_run<true, BF>(p, x - C);
}

// ---------------------------------------------------------------------------
// k_bw_grads: the chunk-wide products of the parameter gradients.  With
// S0 = S_c, dSC = dS_{c+1}:
//   U = U0 - W S0 ; dU = M^T dO + Kc dSC ; dX = T^T dU ; dv = dX w ; dw = dX v
//   dM = mask(dO U^T), dA = -mask(dX U^T)            -> workspace
//   U dSC^T, dO S0^T, dX S0^T -> workspace (Rk, Rq, Rb; k_bw_dqk finishes dk, dq, db)
// Wave w owns the columns 16w..16w+15 of every C x 128 product.
// ---------------------------------------------------------------------------
// a 64 x 16 product tile of wave wv in accumulator order: one 16-byte
// vector per lane and row block
__device__ __forceinline__ void store_frag(float* R, int wv, int l, const f32x4 (&acc)[4][TPW]) {
#pragma unroll
  for (int I = 0; I < 4; ++I)
    *reinterpret_cast<float4*>(R + ((wv * 4 + I) * 64 + l) * 4) = make_float4(acc[I][0][0], acc[I][0][1], acc[I][0][2], acc[I][0][3]);
}

__device__ __forceinline__ void zero_acc(f32x4 (&acc)[4][TPW]) {
#pragma unroll
  for (int I = 0; I < 4; ++I)
#pragma unroll
    for (int R2 = 0; R2 < TPW; ++R2) acc[I][R2] = zero4();
}

// this lane's rows of a product's right operand (Y rows 16 w + l16, all 128
// columns), loaded ahead of the product
__device__ __forceinline__ void load_y(float (&y)[4][8], const float* Y, int wv, int q, int l16) {
#pragma unroll
  for (int s = 0; s < 4; ++s) row8(Y + (16 * wv + l16) * KD, s, q, y[s]);
}

// the same operand rows of Y = X^T, read from row-major X: column 16 w + l16
// of X, rows 32 s + pi_k(q, e)
__device__ __forceinline__ void load_yT(float (&y)[4][8], const float* X, int wv, int q, int l16) {
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int e = 0; e < 8; ++e) y[s][e] = X[(32 * s + pi_k(q, e)) * KD + 16 * wv + l16];
}

// A 64 x W matrix in LDS: fp32, or in bf16 mode split into high and low
// bf16 planes (the same bytes), so that the split products read their
// operands without converting them: each value is split once, by the thread
// that stores it, instead of by every wave that reads it.
template <bool BF, int W> struct LMat;
template <int W> struct LMat<false, W> {
  alignas(16) float a[BC][W + 4];
  __device__ __forceinline__ Frag<false> row_frag(int r, int s, int q) const {
    float x[8];
    row8(&a[r][0], s, q, x);
    return fr8(x);
  }
  // column c, rows 32 s + pi_k(q, e)
  __device__ __forceinline__ Frag<false> col_frag(int c, int s, int q) const {
    float x[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = a[32 * s + pi_k(q, e)][c];
    return fr8(x);
  }
  __device__ __forceinline__ void put(int r, int c, float v) { a[r][c] = v; }
  __device__ __forceinline__ void put4(int r, int c, float4 v) { *reinterpret_cast<float4*>(&a[r][c]) = v; }
  __device__ __forceinline__ float4 get4(int r, int c) const { return *reinterpret_cast<const float4*>(&a[r][c]); }
};
template <int W> struct LMat<true, W> {
  alignas(16) bf16 h[BC][W + 4];   // rows of (W + 4) * 2 bytes: 8-byte vector access at c % 4 == 0
  alignas(16) bf16 lw[BC][W + 4];
  __device__ __forceinline__ Pol<true>::F3 row_frag(int r, int s, int q) const {
    Pol<true>::F3 f;
    const bf16x4 h0 = *reinterpret_cast<const bf16x4*>(&h[r][32 * s + 4 * q]);
    const bf16x4 h1 = *reinterpret_cast<const bf16x4*>(&h[r][32 * s + 16 + 4 * q]);
    const bf16x4 l0 = *reinterpret_cast<const bf16x4*>(&lw[r][32 * s + 4 * q]);
    const bf16x4 l1 = *reinterpret_cast<const bf16x4*>(&lw[r][32 * s + 16 + 4 * q]);
    f.hi.v = bf16x8{h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
    f.lo.v = bf16x8{l0[0], l0[1], l0[2], l0[3], l1[0], l1[1], l1[2], l1[3]};
    return f;
  }
  __device__ __forceinline__ Pol<true>::F3 col_frag(int c, int s, int q) const {
    Pol<true>::F3 f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      f.hi.v[e] = h[32 * s + pi_k(q, e)][c];
      f.lo.v[e] = lw[32 * s + pi_k(q, e)][c];
    }
    return f;
  }
  __device__ __forceinline__ void put(int r, int c, float v) {
    const bf16 x = (bf16)v;
    h[r][c] = x;
    lw[r][c] = (bf16)(v - (float)x);
  }
  __device__ __forceinline__ void put4(int r, int c, float4 v) {
    const float x[4] = {v.x, v.y, v.z, v.w};
    bf16x4 hh, ll;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      hh[e] = (bf16)x[e];
      ll[e] = (bf16)(x[e] - (float)hh[e]);
    }
    *reinterpret_cast<bf16x4*>(&h[r][c]) = hh;
    *reinterpret_cast<bf16x4*>(&lw[r][c]) = ll;
  }
  __device__ __forceinline__ float4 get4(int r, int c) const {
    const bf16x4 hh = *reinterpret_cast<const bf16x4*>(&h[r][c]);
    const bf16x4 ll = *reinterpret_cast<const bf16x4*>(&lw[r][c]);
    return make_float4((float)hh[0] + (float)ll[0], (float)hh[1] + (float)ll[1], (float)hh[2] + (float)ll[2],
                       (float)hh[3] + (float)ll[3]);
  }
};

// acc[I] += X[rows 16I..][:] * Y^T with X in LDS and Y's fragments preloaded
template <bool BF>
__device__ __forceinline__ void nt_lds(f32x4 (&acc)[4][TPW], const LMat<BF, KD>& X,
                                       const typename Op<BF>::F (&y)[4], int q, int l16) {
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int I = 0; I < 4; ++I) Op<BF>::mac(acc[I][0], X.row_frag(16 * I + l16, s, q), y[s]);
}
template <bool BF>
__device__ __forceinline__ void split4(const float (&y)[4][8], typename Op<BF>::F (&f)[4]) {
#pragma unroll
  for (int s = 0; s < 4; ++s) f[s] = Op<BF>::make(y[s]);
}

// Every operand that comes from global memory is loaded one phase ahead of
// its product (state rows into registers; W, Kc and M^T staged in LDS), so
// each phase waits on at most the loads issued a phase earlier.
template <bool BF>
__global__ __launch_bounds__(NT) void k_bw_grads(BW p) {
  using O = Op<BF>;
  __shared__ LMat<BF, KD> sdO, sX, sU, sT;   // sX: dU, then dX; sT: W, then Kc
  __shared__ LMat<BF, BC> sMT;               // M^T, then T^T
  __shared__ int sseg[BC], scar[BC], slast[BC];
  static_assert(TPW == 1, "one 16-column tile per wave");

  const int u = blockIdx.x;
  const int c = u % p.NC, bh = u / p.NC, h = bh % p.H, bb = bh / p.H;
  const int t0 = (p.c0 + c) * BC;
  const int tid = threadIdx.x, l = tid & 63, wv = tid >> 6, q = l >> 4, l16 = l & 15;
  const int vcol = 16 * wv + l16;
  const float* S0 = p.S + (int64_t)u * KK;
  const float* dSC = p.dS + (int64_t)u * KK;

  if (tid < BC) chunk_docs(p, bb, t0, sseg, scar, slast);
  float yA[4][8], yB[4][8], yS0[4][8];
  load_y(yA, S0, wv, q, l16);
  load_yT(yS0, S0, wv, q, l16);
  float4 u0[4];
#pragma unroll
  for (int I = 0; I < 4; ++I) u0[I] = ld4g(p.U0T + (int64_t)u * CK + aofs(vcol, 16 * I + 4 * q, BC / 16));
#pragma unroll
  for (int it = 0; it < BC * KD / 4 / NT; ++it) {
    const int idx = tid + NT * it, i = idx / (KD / 4), c4 = idx % (KD / 4);
    const float4 v = t0 + i < p.L ? ld4_dt(p.dout, row_of(p, bb, t0 + i, h) + 4 * c4, p.dout_dt) : zero_f4();
    sdO.put4(i, 4 * c4, v);
  }
  // W (then Kc below) from the scan operand order: per task one lane's run pair
  auto stage_op = [&](const float* arr, LMat<BF, KD>& dstT) {
    for (int task = tid; task < BC * KD / 8; task += NT) {
      const int ln = task & 63, pr = task >> 6, blk = pr / (KD / 32), s = pr % (KD / 32);
      const int i = 16 * blk + (ln & 15), cc = 32 * s + 4 * (ln >> 4);
      float x[8];
      op_get8<BF>(arr, i, cc, KD / 32, x);
      dstT.put4(i, cc, make_float4(x[0], x[1], x[2], x[3]));
      dstT.put4(i, cc + 16, make_float4(x[4], x[5], x[6], x[7]));
    }
  };
  stage_op(p.Wm + (int64_t)u * CK, sT);
#pragma unroll
  for (int it = 0; it < CC / 4 / NT; ++it) {
    const int idx = tid + NT * it, i = idx / (BC / 4), c4 = idx % (BC / 4);
    sMT.put4(i, 4 * c4, ld4g(p.MT + (int64_t)u * CC + i * BC + 4 * c4));
  }
  lds_barrier();

  f32x4 acc[4][TPW];
  // ---- U = U0 - W S0 ---------------------------------------------------------
  zero_acc(acc);
  typename O::F fA[4], fS0[4], fB[4];
  split4<BF>(yA, fA);
  nt_lds<BF>(acc, sT, fA, q, l16);
  load_yT(yB, dSC, wv, q, l16);
  // Kc: this thread's two run-pair lanes, staged once W is done
  static_assert(BC * KD / 8 == 2 * NT, "two run-pair lanes per thread");
  float kcx[2][8];
  auto kc_pos = [&](int t2, int& i, int& cc) {
    const int task = tid + NT * t2, ln = task & 63, pr = task >> 6;
    i = 16 * (pr / (KD / 32)) + (ln & 15);
    cc = 32 * (pr % (KD / 32)) + 4 * (ln >> 4);
  };
#pragma unroll
  for (int t2 = 0; t2 < 2; ++t2) {
    int i, cc;
    kc_pos(t2, i, cc);
    op_get8<BF>(p.Kc + (int64_t)u * CK, i, cc, KD / 32, kcx[t2]);
  }
#pragma unroll
  for (int I = 0; I < 4; ++I)
#pragma unroll
    for (int e = 0; e < 4; ++e) sU.put(16 * I + 4 * q + e, vcol, f4at(u0[I], e) - acc[I][0][e]);
  lds_barrier();   // U complete; every wave is done with W
#pragma unroll
  for (int t2 = 0; t2 < 2; ++t2) {
    int i, cc;
    kc_pos(t2, i, cc);
    sT.put4(i, cc, make_float4(kcx[t2][0], kcx[t2][1], kcx[t2][2], kcx[t2][3]));
    sT.put4(i, cc + 16, make_float4(kcx[t2][4], kcx[t2][5], kcx[t2][6], kcx[t2][7]));
  }

  // rowsum over v of S0 * dSC for channel 16 wv + l16 (the lane's S0 and dSC
  // columns hold the same (k, v) pairs; the 4 lanes of a channel split v)
  {
    float rs = 0.f;
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) rs += yS0[s][e] * yB[s][e];
    rs += __shfl_xor(rs, 16);
    rs += __shfl_xor(rs, 32);
    if (q == 0) p.RS[(int64_t)u * KD + vcol] = rs;
  }
  // ---- U dSC^T (Kc part of dk, raw) and dO S0^T (dq, raw) -------------------
  load_y(yA, dSC, wv, q, l16);
  split4<BF>(yB, fB);
  split4<BF>(yS0, fS0);
  zero_acc(acc);
  nt_lds<BF>(acc, sU, fB, q, l16);
  store_frag(p.Rk + (int64_t)u * CK, wv, l, acc);
  zero_acc(acc);
  nt_lds<BF>(acc, sdO, fS0, q, l16);
  store_frag(p.Rq + (int64_t)u * CK, wv, l, acc);
  // T^T (64 x 64, row-major) for the dX phase: loaded once per workgroup
  // (two 16-byte pieces per thread), staged into M^T's LDS once dU is done
  static_assert(CC / 4 == 2 * NT, "two float4 of T^T per thread");
  float4 ttq[2];
#pragma unroll
  for (int it = 0; it < 2; ++it) ttq[it] = ld4g(p.TT + (int64_t)u * CC + 4 * (tid + NT * it));
  // w, v of the coalesced dv / dw pass: float4s tid + NT it of the chunk's
  // row-major 64 x 128 tiles
  float4 wq[BC * KD / 4 / NT], vq[BC * KD / 4 / NT];
#pragma unroll
  for (int it = 0; it < BC * KD / 4 / NT; ++it) {
    const int idx = tid + NT * it, i = idx / (KD / 4), c4 = idx % (KD / 4);
    const bool vi = t0 + i < p.L;
    const int64_t ro = row_of(p, bb, vi ? t0 + i : 0, h) + 4 * c4;
    wq[it] = vi ? ld4g(p.w + ro) : zero_f4();
    vq[it] = vi ? ld4_dt(p.v, ro, p.v_dt) : zero_f4();
  }
  lds_barrier();   // Kc staged

  // ---- dU = M^T dO + Kc dSC  (into sX) --------------------------------------
  zero_acc(acc);
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const typename O::F bfr = sdO.col_frag(vcol, s, q);
#pragma unroll
    for (int I = 0; I < 4; ++I)
      if (s == 1 || I < 2) O::mac(acc[I][0], sMT.row_frag(16 * I + l16, s, q), bfr);   // M^T / T^T upper triangular
  }
  split4<BF>(yA, fA);
  nt_lds<BF>(acc, sT, fA, q, l16);
#pragma unroll
  for (int I = 0; I < 4; ++I)
#pragma unroll
    for (int e = 0; e < 4; ++e) sX.put(16 * I + 4 * q + e, vcol, acc[I][0][e]);
  lds_barrier();   // dU complete; every wave is done with M^T
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int idx = tid + NT * it;
    sMT.put4(idx / (BC / 4), 4 * (idx % (BC / 4)), ttq[it]);
  }
  lds_barrier();

  // ---- dX = T^T dU ; dv = dX w ; dw = dX v ----------------------------------
  zero_acc(acc);
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const typename O::F bfr = sX.col_frag(vcol, s, q);
#pragma unroll
    for (int I = 0; I < 4; ++I)
      if (s == 1 || I < 2) O::mac(acc[I][0], sMT.row_frag(16 * I + l16, s, q), bfr);   // M^T / T^T upper triangular
  }
  lds_barrier();
#pragma unroll
  for (int I = 0; I < 4; ++I)
#pragma unroll
    for (int e = 0; e < 4; ++e) sX.put(16 * I + 4 * q + e, vcol, acc[I][0][e]);
  lds_barrier();
  // dv = dX w, dw = dX v, row-major and coalesced
#pragma unroll
  for (int it = 0; it < BC * KD / 4 / NT; ++it) {
    const int idx = tid + NT * it, i = idx / (KD / 4), c4 = idx % (KD / 4);
    if (t0 + i < p.L) {
      const int64_t ro = row_of(p, bb, t0 + i, h) + 4 * c4;
      const float4 dx = sX.get4(i, 4 * c4);
      const float4 a = wq[it], v4 = vq[it];
      const float4 dv = make_float4(dx.x * a.x, dx.y * a.y, dx.z * a.z, dx.w * a.w);
      if (p.dv_dt == DT_BF16) {
        bf16x4 hb;
        hb[0] = (bf16)dv.x; hb[1] = (bf16)dv.y; hb[2] = (bf16)dv.z; hb[3] = (bf16)dv.w;
        *reinterpret_cast<bf16x4*>(reinterpret_cast<bf16*>(p.dv) + ro) = hb;
      } else {
        *reinterpret_cast<float4*>(p.dv + ro) = dv;
      }
      *reinterpret_cast<float4*>(p.dw + ro) = make_float4(dx.x * v4.x, dx.y * v4.y, dx.z * v4.z, dx.w * v4.w);
    }
  }

  // ---- dX S0^T (the initial-state part of dbeta, raw) -----------------------
  zero_acc(acc);
  nt_lds<BF>(acc, sX, fS0, q, l16);
  store_frag(p.Rb + (int64_t)u * CK, wv, l, acc);

  // ---- dM = mask(dO U^T), dA = -mask(dX U^T), to the workspace -------------
  // The 10 lower-triangle 16 x 16 tiles of each (20 products, at most three
  // per wave); the 6 tiles above the diagonal are zero.
  for (int task = wv; task < 20; task += NWV) {
    const bool isA = task >= 10;
    const int tt = task % 10;
    const int I = (tt >= 1) + (tt >= 3) + (tt >= 6);
    const int J = tt - I * (I + 1) / 2;
    float* dst = (isA ? p.dAw : p.dMw) + (int64_t)u * CC;
    f32x4 a = zero4();
    const LMat<BF, KD>& Xs = isA ? sX : sdO;
#pragma unroll
    for (int s = 0; s < 4; ++s) O::mac(a, Xs.row_frag(16 * I + l16, s, q), sU.row_frag(16 * J + l16, s, q));
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 16 * I + 4 * q + e, j = 16 * J + l16;
      const bool ok = (isA ? j < i : j <= i) && sseg[i] == sseg[j];
      dst[i * BC + j] = ok ? (isA ? -a[e] : a[e]) : 0.f;
    }
  }
  for (int idx = tid; idx < 2 * 6 * 64; idx += NT) {   // float4s of the upper tiles
    const int m = idx / (6 * 64), t = (idx / 64) % 6, f4 = idx % 64;
    const int I = t < 3 ? 0 : (t < 5 ? 1 : 2), J = t < 3 ? t + 1 : (t < 5 ? t - 1 : 3);
    float* dst = (m ? p.dAw : p.dMw) + (int64_t)u * CC;
    *reinterpret_cast<float4*>(dst + (16 * I + f4 / 4) * BC + 16 * J + 4 * (f4 % 4)) = zero_f4();
  }
}

// ---------------------------------------------------------------------------
// k_bw_dqk: the decay-weighted parts of dq, dbeta, dk and dg, per (unit,
// quarter of the key channels).  With the chunk's q, k, b, G and dM, dA in LDS:
//   dq_i    = carry_i e^{G_i} (dO S0^T)_i + sum_j dM_ij e^{G_i-G_j} k_j
//   dbeta_i = -carry_i e^{G_i} (dX S0^T)_i + sum_j dA_ij e^{G_i-G_j} k_j
//   dk_j    = sum_i dM_ij e^{G_i-G_j} q_i + sum_i dA_ij e^{G_i-G_j} beta_i
//             + last_j e^{G_last-G_j} (U dSC^T)_j
//   dG_i    = q_i dq_i + beta_i dbeta_i - k_i dk_i   (pairs whose factor is e^0
//             left out: they cancel), db = k dbeta, dk += b dbeta,
//   dg_t    = sum_{i>=t} dG_i + sum_{j<t} k_j dk_j^(Kc) + lam rowsum(S0 * dSC)
// Off-diagonal 16-row blocks use e^{G_i-G_m} e^{G_m-G_j} (both <= 1) through
// MFMA; pairs inside a block join those products where the block's decay
// span allows, else use e^{G_i-G_j} per element.
// Wave w owns the 16 channels 16 (w % 2) .. and the 16-row block w / 2;
// lanes hold rows 4q..4q+3 of it.  About 73 KB of LDS: two workgroups per CU.
// ---------------------------------------------------------------------------
constexpr int HC = KD / 4;      // channels per k_bw_dqk workgroup
constexpr int NQ = KD / HC;     // k_bw_dqk workgroups per unit
constexpr int HP = HC + 4;

// fp32 product over half of a fragment's k elements (4 h .. 4 h + 3), for
// operands whose other half is zero
__device__ __forceinline__ void mma_half(f32x4& acc, const float* a, const float* b, int h) {
  if (h) {
#pragma unroll
    for (int e = 4; e < 8; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], b[e], acc, 0, 0, 0);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], b[e], acc, 0, 0, 0);
  }
}

__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(4))) void k_bw_dqk(BW p) {
  __shared__ float sQ[BC][HP], sK[BC][HP], sB[BC][HP], sG[BC][HP];
  __shared__ float sdM[BC][CP], sdA[BC][CP];
  __shared__ float sSegP[NT / HC][HC], sSegG[NT / HC][HC];   // 4-token segment sums of P and dG
  __shared__ int scar[BC], slast[BC], sseg[BC];

  const int u = blockIdx.x / NQ, part = blockIdx.x % NQ;
  const int c = u % p.NC, bh = u / p.NC, h = bh % p.H, bb = bh / p.H;
  const int t0 = (p.c0 + c) * BC;
  const int tid = threadIdx.x, l = tid & 63, wv = tid >> 6, q = l >> 4, l16 = l & 15;
  const int ch0 = HC * part;
  const float* G = p.G + (int64_t)u * CK;

  constexpr int CG = HC / 16;                // 16-channel groups
  constexpr int NB = 4 * CG / NWV;           // 16-row blocks per wave
  const int rl = 16 * (wv % CG) + l16, r = ch0 + rl;
  const int I0 = NB * (wv / CG);
  // raw products from k_bw_grads for this lane's rows, loaded up front
  // (k_bw_grads stored them in accumulator order: column tile r / 16, the
  // same lane, rows 16 I + 4 q + e; rows past the sequence end count as zero)
  float rq[NB][4], rb[NB][4], rk[NB][4];
#pragma unroll
  for (int Ib = 0; Ib < NB; ++Ib) {
    const int I = I0 + Ib;
    const int64_t fo = (int64_t)u * CK + (((r >> 4) * 4 + I) * 64 + l) * 4;
    const float4 fq = ld4g(p.Rq + fo), fb = ld4g(p.Rb + fo), fk = ld4g(p.Rk + fo);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool vi = t0 + 16 * I + 4 * q + e < p.L;
      rq[Ib][e] = vi ? f4at(fq, e) : 0.f;
      rb[Ib][e] = vi ? f4at(fb, e) : 0.f;
      rk[Ib][e] = vi ? f4at(fk, e) : 0.f;
    }
  }
  // rowsum(S0 * dSC) of the thread's channel, formed by k_bw_grads
  const float rsum = p.RS[(int64_t)u * KD + ch0 + tid % HC];
  if (tid < BC) chunk_docs(p, bb, t0, sseg, scar, slast);
#pragma unroll
  for (int it = 0; it < BC * HC / 4 / NT; ++it) {
    const int idx = tid + NT * it, i = idx / (HC / 4), c4 = idx % (HC / 4);
    float4 qv = zero_f4(), kv = zero_f4(), bv = zero_f4();
    if (t0 + i < p.L) {
      const int64_t rq = row_in(p, bb, t0 + i, h, p.qk_hd) + ch0 + 4 * c4;
      qv = ld4g(p.q + rq); kv = ld4g(p.k + rq); bv = ld4g(p.b + row_in(p, bb, t0 + i, h, p.gb_hd) + ch0 + 4 * c4);
    }
    *reinterpret_cast<float4*>(&sQ[i][4 * c4]) = qv;
    *reinterpret_cast<float4*>(&sK[i][4 * c4]) = kv;
    *reinterpret_cast<float4*>(&sB[i][4 * c4]) = bv;
    *reinterpret_cast<float4*>(&sG[i][4 * c4]) = ld4g(G + i * KD + ch0 + 4 * c4);
  }
#pragma unroll
  for (int it = 0; it < CC / 4 / NT; ++it) {
    const int idx = tid + NT * it, i = idx / (BC / 4), c4 = idx % (BC / 4);
    *reinterpret_cast<float4*>(&sdM[i][4 * c4]) = ld4g(p.dMw + (int64_t)u * CC + i * BC + 4 * c4);
    *reinterpret_cast<float4*>(&sdA[i][4 * c4]) = ld4g(p.dAw + (int64_t)u * CC + i * BC + 4 * c4);
  }
  lds_barrier();

  const float glast = sG[BC - 1][rl];
  float rdg[NB][4], rpp[NB][4];   // dG and P of this lane's rows
#pragma unroll
  for (int Ib = 0; Ib < NB; ++Ib) {
    const int I = I0 + Ib;
    // rows i of block I against columns j < 16 I (and, for dk, rows j of the
    // block against i > 16 I + 15) through MFMA.  Where the block's decay span
    // stays below 2^64 in this wave's channels (and it holds one document),
    // the pairs inside the block join the dq / dbeta products: their column
    // factor e^{G_m - G_j} is then >= 1 and bounded.  The pair (i, i) is left
    // out of dq and dk (its factor is e^0).
    // dk's pairs inside block I are scaled from the block's first row m (<= i)
    // in their own accumulator, okb (factor e^{G_j - G_m} <= 1, then
    // e^{G_m - G_i} <= 2^64): a factor through the last row m2 would round
    // differently with the decays of tokens after i, and a loss on tokens
    // before some t must give their gradients bit for bit whatever follows t
    // (the reference's tests/test_causality.py)
    f32x4 oq = zero4(), ob = zero4(), ok_ = zero4(), okb = zero4();
    const int m = 16 * I, m2 = 16 * I + 15;
    const float gm = sG[m][rl], gm2 = sG[m2][rl];
    // G restarts at document starts: the in-block factors need one document
    const bool inblk = sseg[m] == sseg[m2] && __all(gm - gm2 <= 64.f);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      float xm[8], xa[8], xk[8], ym[8], ya[8], yq[8], yb[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        // the 16-row block of column j is known here; I is the same in the
        // whole wave, so which side of block I it lies on is a uniform branch
        const int jb = 2 * s + (e >> 2);
        const int j = 32 * s + pi_k(q, e);
        const float gj = sG[j][rl];
        if (jb < I) {
          xm[e] = sdM[16 * I + l16][j];
          xa[e] = sdA[16 * I + l16][j];
          xk[e] = sK[j][rl] * ex2(gm - gj);
          ym[e] = ya[e] = yq[e] = yb[e] = 0.f;
        } else if (jb > I) {
          xm[e] = xa[e] = xk[e] = 0.f;
          ym[e] = sdM[j][16 * I + l16];
          ya[e] = sdA[j][16 * I + l16];
          const float f = ex2(gj - gm2);
          yq[e] = sQ[j][rl] * f;
          yb[e] = sB[j][rl] * sK[j][rl] * f;
        } else if (inblk) {
          const bool self = j == 16 * I + l16;
          xm[e] = self ? 0.f : sdM[16 * I + l16][j];
          xa[e] = sdA[16 * I + l16][j];
          xk[e] = sK[j][rl] * __builtin_amdgcn_exp2f(gm - gj);
          ym[e] = ya[e] = yq[e] = yb[e] = 0.f;   // dk's in-block pairs: okb below
        } else {
          xm[e] = xa[e] = xk[e] = ym[e] = ya[e] = yq[e] = yb[e] = 0.f;
        }
      }
      // slab s holds row blocks 2s and 2s + 1: a side with no column in it
      // has all-zero operands (a uniform test: I is the wave's block)
      const bool any_lo = 2 * s < I || (inblk && I / 2 == s);
      const bool any_hi = 2 * s + 1 > I;
      // in the slab of block I (2 s == I: blocks I, I + 1) only one half of
      // the k elements is nonzero on each side
      if (any_lo) {
        if (2 * s == I) {
          mma_half(oq, xm, xk, 0);
          mma_half(ob, xa, xk, 0);
        } else {
          const Frag<false> fk = fr8(xk);
          mma(oq, fr8(xm), fk);
          mma(ob, fr8(xa), fk);
        }
      }
      if (any_hi) {
        if (2 * s == I) {
          mma_half(ok_, ym, yq, 1);
          mma_half(ok_, ya, yb, 1);
        } else {
          mma(ok_, fr8(ym), fr8(yq));
          mma(ok_, fr8(ya), fr8(yb));
        }
      }
    }
    if (inblk) {   // dk's pairs inside block I: slab I / 2, elements of block I
      const int s = I / 2;
      float zm[8], za[8], zq[8], zb[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int jb = 2 * s + (e >> 2);
        const int j = 32 * s + pi_k(q, e);
        if (jb == I) {
          const bool self = j == 16 * I + l16;
          zm[e] = self ? 0.f : sdM[j][16 * I + l16];
          za[e] = sdA[j][16 * I + l16];
          const float f = __builtin_amdgcn_exp2f(sG[j][rl] - gm);   // <= 1: one document, G monotone
          zq[e] = sQ[j][rl] * f;
          zb[e] = sB[j][rl] * sK[j][rl] * f;
        } else {
          zm[e] = za[e] = zq[e] = zb[e] = 0.f;
        }
      }
      mma_half(okb, zm, zq, I & 1);   // block I is half I & 1 of slab I / 2
      mma_half(okb, za, zb, I & 1);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int ii = 4 * q + e;
      const int i = 16 * I + ii;
      const float gi = sG[i][rl];
      float dq = 0.f, dbeta = 0.f, dk = 0.f;
      if (!inblk) {
        // pairs inside block I, e^{G_i - G_j} per element
#pragma unroll
        for (int jj = 0; jj < 16; ++jj) {
          const int j = 16 * I + jj;
          const float kj = sK[j][rl], gj = sG[j][rl];
          const float off = jj == ii ? 0.f : 1.f;
          const float fij = ex2(gi - gj);
          dq += off * sdM[i][j] * fij * kj;
          dbeta += sdA[i][j] * fij * kj;
          const float fji = ex2(gj - gi);
          dk += off * sdM[j][i] * fji * sQ[j][rl] + sdA[j][i] * fji * (sB[j][rl] * kj);
        }
      }
      const float eg = scar[i] ? ex2(gi) : 0.f;
      dq += eg * rq[Ib][e] + oq[e] * ex2(gi - gm);
      dbeta += -eg * rb[Ib][e] + ob[e] * ex2(gi - gm);
      dk += ok_[e] * ex2(gm2 - gi);
      if (inblk) dk += okb[e] * __builtin_amdgcn_exp2f(gm - gi);   // <= 2^64 (the block's span)
      const float dkc = slast[i] ? ex2(glast - gi) * rk[Ib][e] : 0.f;
      const float kv = sK[i][rl], qv = sQ[i][rl], bv = sB[i][rl], dmii = sdM[i][i];
      rdg[Ib][e] = qv * dq + bv * kv * dbeta - kv * dk;
      rpp[Ib][e] = kv * dkc;
      if (t0 + i < p.L) {
        const int64_t ro = row_of(p, bb, t0 + i, h) + r;
        p.dq[ro] = dq + dmii * kv;
        p.dk[ro] = dk + dmii * qv + dkc + bv * dbeta;
        p.db[ro] = kv * dbeta;
      }
    }
  }
  // dG and P rows replace q and k in LDS once every wave is done with them
  lds_barrier();
  float (*sdG)[HP] = sQ;
  float (*sP)[HP] = sK;
#pragma unroll
  for (int Ib = 0; Ib < NB; ++Ib)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 16 * (I0 + Ib) + 4 * q + e;
      sdG[i][rl] = rdg[Ib][e];
      sP[i][rl] = rpp[Ib][e];
    }
  lds_barrier();

  // ---- dg_t = sum_{i>=t} dG_i + sum_{j<t} P_j + lam rowsum(S0 * dSC) -------
  // (the Kc pair (j, last) enters dg_t for t <= j twice with opposite signs,
  // so it is summed forward over j < t instead)
  // Every thread: channel tid % HC, tokens 4 sg .. 4 sg + 3; the segment
  // sums go through LDS, then each thread scans its own four tokens.
  {
    constexpr int NSG = NT / HC;
    static_assert(4 * NSG == BC, "one 4-token segment per thread");
    const int ch = tid % HC, sg = tid / HC;
    float pl[4], gl[4], ps = 0.f, gs = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      pl[e] = sP[4 * sg + e][ch];
      gl[e] = sdG[4 * sg + e][ch];
      ps += pl[e];
      gs += gl[e];
    }
    sSegP[sg][ch] = ps;
    sSegG[sg][ch] = gs;
    lds_barrier();
    float fwd = 0.f, acc = scar[BC - 1] ? ex2(sG[BC - 1][ch]) * rsum : 0.f;
#pragma unroll
    for (int s2 = 0; s2 < NSG; ++s2) {
      if (s2 < sg) fwd += sSegP[s2][ch];
      if (s2 > sg) acc += sSegG[s2][ch];
    }
    float dgv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      dgv[e] = fwd;
      fwd += pl[e];
    }
#pragma unroll
    for (int e = 3; e >= 0; --e) {
      acc += gl[e];
      dgv[e] += acc;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (t0 + 4 * sg + e < p.L) p.dg[row_of(p, bb, t0 + 4 * sg + e, h) + ch0 + ch] = dgv[e];
  }
}

// ---------------------------------------------------------------------------
// Raw-input backward: the whole training op's VJP from the forward's own
// arguments (dn_prefill_args): segment canonicalisation, the wrapper's
// prologue (gdn2.py:1970-2125, 133-142) recomputed per value head, the
// recurrence backward above, and the prologue's derivatives summed back to
// each raw layout (GQA groups, broadcast gate heads / channels).
// ---------------------------------------------------------------------------
struct BR {
  int B, L, Hk, Hv, G;
  const void *q, *k, *v;
  int qk_dt, v_dt;
  const float *g, *b, *w;
  int g_h, g_c, b_h, b_c, w_h, w_c;
  const void* seg; int seg_dt, seg_batched;
  const int32_t* init_seg; int has_init;
  float scale; int l2norm, fuse, guard;
  int32_t* canon;                                 // (B, L)
  float *qe, *ke, *ve, *ge, *be, *we;             // prepared inputs: qe, ke (B, L, Hk, 128); ge, be
                                                  // (B, L, Hv / gb_hd, 128); ve, we (B, L, Hv, 128)
  int gb_hd;                                      // G when g and b both sit at the key heads, else 1
  int w_alias;                                    // w's prologue step is the identity: we unused
  const float *dqe, *dke, *dge, *dbe, *dwe;       // their gradients
  float *dq, *dk, *dg, *db, *dw;                  // raw-layout gradients (dq, dk in qk_dt)
};

__device__ __forceinline__ int gate_head(int H, int Hk, int Hv, int hv, int G) {
  return H == Hv ? hv : (H == Hk ? hv / G : 0);
}
__device__ __forceinline__ float sigmoid_hw(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }
// sigmoid'(x) = s(x) s(-x) = e s^2 with e = e^{-|x|}, s = 1 / (1 + e): no
// 1 - s(x), which loses the low bits once s(x) nears 1 (at x = 10, 1 - s is
// 4.5e-5 and fp32 keeps it to ~1e-3 relative)
__device__ __forceinline__ float dsigmoid(float x) {
  const float e = __expf(-fabsf(x));
  const float s = __builtin_amdgcn_rcpf(1.f + e);
  return e * s * s;
}

// canonical ids: first_new + number of changes in seg[1..t] (gdn2.py:2081-2094),
// batch row bb by one workgroup of NT threads
template <int NT>
__device__ __forceinline__ void canon_rows(const BR& p, int bb) {
  constexpr int NWc = NT / 64;
  __shared__ int wsum[NWc];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t base = p.seg_batched ? (int64_t)bb * p.L : 0;
  auto sid = [&](int t) -> int64_t { return p.seg ? ld_i(p.seg, base + t, p.seg_dt) : 0; };
  // tiles of NT tokens: thread tid flags token ts + tid as a change from the
  // token before it; a block-wide inclusive scan of the flags gives the ids
  int run = (p.has_init && p.init_seg != nullptr) ? (sid(0) != (int64_t)p.init_seg[bb]) : 0;
  for (int ts = 0; ts < p.L; ts += NT) {
    const int t = ts + tid;
    int f = (t > 0 && t < p.L) ? (sid(t) != sid(t - 1)) : 0;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int x = __shfl_up(f, o);
      if (lane >= o) f += x;
    }
    if (lane == 63) wsum[wid] = f;
    __syncthreads();
    int before = run, tile = 0;
#pragma unroll
    for (int w = 0; w < NWc; ++w) {
      before += w < wid ? wsum[w] : 0;
      tile += wsum[w];
    }
    if (t < p.L) p.canon[(int64_t)bb * p.L + t] = before + f;
    run += tile;
    __syncthreads();   // wsum is rewritten by the next tile
  }
}

// four consecutive elements of an f32 / bf16 / f16 array
__device__ __forceinline__ void ld4_any(const void* p, int64_t i, int dt, float* x) {
  if (dt == DT_BF16) {
    const bf16x4 v = *reinterpret_cast<const bf16x4*>((const bf16*)p + i);
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = (float)v[e];
  } else if (dt == DT_F16) {
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = (float)((const f16*)p)[i + e];
  } else {
    const float4 v = ld4g((const float*)p + i);
    x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
  }
}
// four channels c..c+3 of a gate row (one value per head when chans == 1)
__device__ __forceinline__ void gate4(const float* g, int64_t base, int chans, int c, float* x) {
  if (chans == 1) {
    x[0] = x[1] = x[2] = x[3] = g[base];
  } else {
    const float4 v = ld4g(g + base + c);
    x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
  }
}

// Two (batch, token, value head) rows per wave, one per 32-lane half, four
// channels per lane (vector loads and stores): the prepared inputs as the
// forward kernels form them (the L2 norms summed in another order, so the
// last bit can differ).
// The first B workgroups (one per batch row, dispatched first) form the
// canonical segment ids meanwhile.
__global__ __launch_bounds__(256) void k_bw_prep(BR p) {
  if ((int)blockIdx.x < p.B) {
    canon_rows<256>(p, (int)blockIdx.x);
    return;
  }
  const int l = threadIdx.x & 63, c = 4 * (l & 31);
  const int64_t rows = (int64_t)p.B * p.L * p.Hv;
  const int64_t row0 = ((int64_t)(blockIdx.x - p.B) * 4 + (threadIdx.x >> 6)) * 2 + (l >> 5);
  const bool valid = row0 < rows;
  const int64_t row = valid ? row0 : rows - 1;   // both halves take part in the shuffles
  const int hv = (int)(row % p.Hv);
  const int64_t bt = row / p.Hv;
  const int hk = hv / p.G;
  const int64_t qrow = (bt * p.Hk + hk) * KD + c;
  float x[4], y[4];
  ld4_any(p.q, qrow, p.qk_dt, x);
  ld4_any(p.k, qrow, p.qk_dt, y);
  float sq = 0.f, sk = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) { sq += x[e] * x[e]; sk += y[e] * y[e]; }
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) { sq += __shfl_xor(sq, o); sk += __shfl_xor(sk, o); }
  const bool b16 = p.qk_dt != DT_F32;
  const int hg = gate_head(p.g_h, p.Hk, p.Hv, hv, p.G), hb = gate_head(p.b_h, p.Hk, p.Hv, hv, p.G);
  const int hw = gate_head(p.w_h, p.Hk, p.Hv, hv, p.G);
  float gv[4], bv[4], wv[4] = {0.f, 0.f, 0.f, 0.f}, vv[4];
  gate4(p.g, (bt * p.g_h + hg) * p.g_c, p.g_c, c, gv);
  gate4(p.b, (bt * p.b_h + hb) * p.b_c, p.b_c, c, bv);
  if (!p.w_alias) gate4(p.w, (bt * p.w_h + hw) * p.w_c, p.w_c, c, wv);
  ld4_any(p.v, (bt * p.Hv + hv) * KD + c, p.v_dt, vv);
  float qh[4], kh[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if (p.fuse) {
      qh[e] = (x[e] * rsqrtf(sq + 1e-6f)) * p.scale;
      kh[e] = y[e] * rsqrtf(sk + 1e-6f);
    } else if (p.l2norm) {
      qh[e] = (x[e] * rsqrtf(sq + 1e-6f)) * p.scale;
      kh[e] = y[e] * rsqrtf(sk + 1e-6f);
      if (b16) { qh[e] = p.qk_dt == DT_BF16 ? round_as<bf16>(qh[e]) : round_as<f16>(qh[e]);
                 kh[e] = p.qk_dt == DT_BF16 ? round_as<bf16>(kh[e]) : round_as<f16>(kh[e]); }
    } else {
      qh[e] = x[e] * p.scale;
      kh[e] = y[e];
      if (b16) qh[e] = p.qk_dt == DT_BF16 ? round_as<bf16>(qh[e]) : round_as<f16>(qh[e]);
    }
    if (p.fuse) {
      gv[e] = -__expf(fminf(gv[e], 5.f));
      bv[e] = sigmoid_hw(bv[e]);
      wv[e] = sigmoid_hw(wv[e]);
    } else {
      gv[e] = fminf(gv[e], 0.f);
      if (p.guard) bv[e] = fmaxf(bv[e], 0.f);
    }
    if (p.guard) gv[e] = fminf(gv[e], -1e-6f);
  }
  if (!valid) return;
  const int64_t o = row * KD + c;
  // q, k (and g, b at the key heads) once per key head: the first value head
  // of the group writes them
  if (hv % p.G == 0) {
    *reinterpret_cast<float4*>(p.qe + qrow) = make_float4(qh[0], qh[1], qh[2], qh[3]);
    *reinterpret_cast<float4*>(p.ke + qrow) = make_float4(kh[0], kh[1], kh[2], kh[3]);
  }
  if (hv % p.gb_hd == 0) {
    const int64_t og = (bt * (p.Hv / p.gb_hd) + hv / p.gb_hd) * KD + c;
    *reinterpret_cast<float4*>(p.ge + og) = make_float4(gv[0], gv[1], gv[2], gv[3]);
    *reinterpret_cast<float4*>(p.be + og) = make_float4(bv[0], bv[1], bv[2], bv[3]);
  }
  if (!p.w_alias) *reinterpret_cast<float4*>(p.we + o) = make_float4(wv[0], wv[1], wv[2], wv[3]);
  *reinterpret_cast<float4*>(p.ve + o) = make_float4(vv[0], vv[1], vv[2], vv[3]);
}

// two (batch, token, key head) rows per wave, one per 32-lane half, four
// channels per lane: dq, dk through the GQA sum and the L2-norm / scale (a
// bf16 or f16 normalised q / k receives its cotangent in that dtype, as the
// reference's cast back does)
__device__ __forceinline__ void post_qk_rows(const BR& p) {
  const int l = threadIdx.x & 63, c = 4 * (l & 31);
  const int64_t rows = (int64_t)p.B * p.L * p.Hk;
  const int64_t row0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 2 + (l >> 5);
  const bool valid = row0 < rows;
  const int64_t row = valid ? row0 : rows - 1;   // both halves take part in the shuffles
  const int hk = (int)(row % p.Hk);
  const int64_t bt = row / p.Hk;
  float dqh[4] = {0.f, 0.f, 0.f, 0.f}, dkh[4] = {0.f, 0.f, 0.f, 0.f}, x[4], y[4];
  for (int g = 0; g < p.G; ++g) {
    const int64_t er = (bt * p.Hv + hk * p.G + g) * KD + c;
    const float4 a4 = ld4g(p.dqe + er), b4 = ld4g(p.dke + er);
    dqh[0] += a4.x; dqh[1] += a4.y; dqh[2] += a4.z; dqh[3] += a4.w;
    dkh[0] += b4.x; dkh[1] += b4.y; dkh[2] += b4.z; dkh[3] += b4.w;
  }
  const bool b16 = p.qk_dt != DT_F32 && !p.fuse;
  ld4_any(p.q, row * KD + c, p.qk_dt, x);
  ld4_any(p.k, row * KD + c, p.qk_dt, y);
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (b16) {
      dqh[e] = p.qk_dt == DT_BF16 ? round_as<bf16>(dqh[e]) : round_as<f16>(dqh[e]);
      dkh[e] = p.qk_dt == DT_BF16 ? round_as<bf16>(dkh[e]) : round_as<f16>(dkh[e]);
    }
  float dq[4], dk[4];
  if (p.fuse || p.l2norm) {
    float sq = 0.f, sk = 0.f, xq = 0.f, yk = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      sq += x[e] * x[e]; sk += y[e] * y[e];
      xq += x[e] * dqh[e]; yk += y[e] * dkh[e];
    }
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) {
      sq += __shfl_xor(sq, o); sk += __shfl_xor(sk, o);
      xq += __shfl_xor(xq, o); yk += __shfl_xor(yk, o);
    }
    // d/dx of c x / sqrt(|x|^2 + eps) = c r (dx^ - r^2 x (x . dx^))
    const float rq = rsqrtf(sq + 1e-6f), rk = rsqrtf(sk + 1e-6f);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      dq[e] = p.scale * rq * (dqh[e] - rq * rq * x[e] * xq);
      dk[e] = rk * (dkh[e] - rk * rk * y[e] * yk);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) { dq[e] = p.scale * dqh[e]; dk[e] = dkh[e]; }
  }
  if (!valid) return;
  const int64_t o = row * KD + c;
  if (p.qk_dt == DT_BF16) {
    bf16x4 hq, hk4;
#pragma unroll
    for (int e = 0; e < 4; ++e) { hq[e] = (bf16)dq[e]; hk4[e] = (bf16)dk[e]; }
    *reinterpret_cast<bf16x4*>(reinterpret_cast<bf16*>(p.dq) + o) = hq;
    *reinterpret_cast<bf16x4*>(reinterpret_cast<bf16*>(p.dk) + o) = hk4;
  } else if (p.qk_dt == DT_F16) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      reinterpret_cast<f16*>(p.dq)[o + e] = (f16)dq[e];
      reinterpret_cast<f16*>(p.dk)[o + e] = (f16)dk[e];
    }
  } else {
    *reinterpret_cast<float4*>(p.dq + o) = make_float4(dq[0], dq[1], dq[2], dq[3]);
    *reinterpret_cast<float4*>(p.dk + o) = make_float4(dk[0], dk[1], dk[2], dk[3]);
  }
}

__global__ __launch_bounds__(256) void k_bw_post_qk(BR p) { post_qk_rows(p); }

// one thread per raw gate element: the sum of the prepared gradient over the
// value heads and channels it was broadcast to, times the prologue derivative
// derivative of the prologue step of gate WHICH at raw value x
template <int WHICH>
__device__ __forceinline__ float gate_deriv(const BR& p, float x) {
  if (WHICH == 0) {
    if (p.fuse) {
      const float ga = -__expf(fminf(x, 5.f));
      return (x <= 5.f ? -__expf(x) : 0.f) * ((!p.guard || ga <= -1e-6f) ? 1.f : 0.f);
    }
    return (x <= 0.f && (!p.guard || x <= -1e-6f)) ? 1.f : 0.f;
  } else if (WHICH == 1) {
    if (p.fuse) return dsigmoid(x);
    return (!p.guard || x >= 0.f) ? 1.f : 0.f;
  } else {
    if (p.fuse) return dsigmoid(x);
    return 1.f;
  }
}

template <int WHICH>   // 0 = g, 1 = b, 2 = w
__global__ __launch_bounds__(256) void k_bw_post_gate(BR p) {
  const int H = WHICH == 0 ? p.g_h : (WHICH == 1 ? p.b_h : p.w_h);
  const int C = WHICH == 0 ? p.g_c : (WHICH == 1 ? p.b_c : p.w_c);
  const float* raw = WHICH == 0 ? p.g : (WHICH == 1 ? p.b : p.w);
  const float* dpre = WHICH == 0 ? p.dge : (WHICH == 1 ? p.dbe : p.dwe);
  float* out = WHICH == 0 ? p.dg : (WHICH == 1 ? p.db : p.dw);
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t n = (int64_t)p.B * p.L * H * C;
  if (idx >= n) return;
  const int c = (int)(idx % C);
  const int h = (int)((idx / C) % H);
  const int64_t bt = idx / ((int64_t)C * H);
  // value heads that read gate head h: h (H = Hv), h G .. h G + G - 1 (H = Hk), all (H = 1)
  int h0, hn;
  if (H == p.Hv) { h0 = h; hn = 1; }
  else if (H == p.Hk) { h0 = h * p.G; hn = p.G; }
  else { h0 = 0; hn = p.Hv; }
  const float* rowp = dpre + (bt * p.Hv + h0) * KD;
  float s = 0.f;
  if (C == 1) {
    for (int j = 0; j < hn; ++j, rowp += KD) {
      float4 acc = zero_f4();
#pragma unroll 8
      for (int i4 = 0; i4 < KD / 4; ++i4) {
        const float4 x4 = ld4g(rowp + 4 * i4);
        acc.x += x4.x; acc.y += x4.y; acc.z += x4.z; acc.w += x4.w;
      }
      s += (acc.x + acc.y) + (acc.z + acc.w);
    }
  } else {
    for (int j = 0; j < hn; ++j, rowp += KD) s += rowp[c];
  }
  const float x = raw[idx];
  const float d = gate_deriv<WHICH>(p, x);
  out[idx] = s * d;
}

// channel-wise gates (C = 128): one thread per 4 channels of one (token, head)
// row.  Loaded: the row's prepared-gradient sum over the value heads it was
// broadcast to, and its raw values.
struct Gate4 { float4 s, x; };
template <int WHICH>
__device__ __forceinline__ Gate4 post_gate4_load(const BR& p, int64_t row, int c4) {
  const int H = WHICH == 0 ? p.g_h : (WHICH == 1 ? p.b_h : p.w_h);
  const float* raw = WHICH == 0 ? p.g : (WHICH == 1 ? p.b : p.w);
  const float* dpre = WHICH == 0 ? p.dge : (WHICH == 1 ? p.dbe : p.dwe);
  const int h = (int)(row % H);
  const int64_t bt = row / H;
  int h0, hn;
  if (H == p.Hv) { h0 = h; hn = 1; }
  else if (H == p.Hk) { h0 = h * p.G; hn = p.G; }
  else { h0 = 0; hn = p.Hv; }
  const float* rowp = dpre + (bt * p.Hv + h0) * KD + 4 * c4;
  Gate4 r{zero_f4(), ld4g(raw + row * KD + 4 * c4)};
  for (int j = 0; j < hn; ++j, rowp += KD) {
    const float4 x4 = ld4g(rowp);
    r.s.x += x4.x; r.s.y += x4.y; r.s.z += x4.z; r.s.w += x4.w;
  }
  return r;
}
template <int WHICH>
__device__ __forceinline__ void post_gate4_store(const BR& p, int64_t row, int c4, const Gate4& r) {
  float* out = WHICH == 0 ? p.dg : (WHICH == 1 ? p.db : p.dw);
  *reinterpret_cast<float4*>(out + row * KD + 4 * c4) =
      make_float4(r.s.x * gate_deriv<WHICH>(p, r.x.x), r.s.y * gate_deriv<WHICH>(p, r.x.y),
                  r.s.z * gate_deriv<WHICH>(p, r.x.z), r.s.w * gate_deriv<WHICH>(p, r.x.w));
}

template <int WHICH>
__global__ __launch_bounds__(256) void k_bw_post_gate4(BR p) {
  const int H = WHICH == 0 ? p.g_h : (WHICH == 1 ? p.b_h : p.w_h);
  const int64_t row = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
  if (row >= (int64_t)p.B * p.L * H) return;
  const int c4 = threadIdx.x & 31;
  post_gate4_store<WHICH>(p, row, c4, post_gate4_load<WHICH>(p, row, c4));
}

// g and b together when both are channel-wise with the same head count: one
// launch instead of two, both gates' loads issued before either store
__global__ __launch_bounds__(256) void k_bw_post_gate4_gb(BR p) {
  const int64_t row = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
  if (row >= (int64_t)p.B * p.L * p.g_h) return;
  const int c4 = threadIdx.x & 31;
  const Gate4 rg = post_gate4_load<0>(p, row, c4);
  const Gate4 rb = post_gate4_load<1>(p, row, c4);
  post_gate4_store<0>(p, row, c4, rg);
  post_gate4_store<1>(p, row, c4, rb);
}

// dq, dk, dg and db in one launch when g and b are channel-wise at the key
// heads: the same (batch, token, key head) row per 32-lane half in all four
__global__ __launch_bounds__(256) void k_bw_post_qkgb(BR p) {
  const int64_t row = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
  const bool valid = row < (int64_t)p.B * p.L * p.Hk;
  const int c4 = threadIdx.x & 31;
  Gate4 rg{}, rb{};
  if (valid) {
    rg = post_gate4_load<0>(p, row, c4);
    rb = post_gate4_load<1>(p, row, c4);
  }
  post_qk_rows(p);
  if (valid) {
    post_gate4_store<0>(p, row, c4, rg);
    post_gate4_store<1>(p, row, c4, rb);
  }
}

}  // namespace

}  // namespace dn

using namespace dn;

namespace {

constexpr size_t kUnitFloats = 9 * (size_t)CK + 4 * (size_t)CC + 2 * KD + 3 * (size_t)KK;

// Chunks per token block: the whole sequence, or with recompute_states the
// smallest number of chunks that still gives kRecomputeUnits (batch, head,
// chunk) units per launch.
constexpr int kRecomputeUnits = 1024;
int bw_block_chunks(const dn_backward_args* a) {
  const int NC = (a->L + BC - 1) / BC;
  if (!a->recompute_states) return NC;
  const int bh = a->B * a->H;
  return std::min(NC, std::max(1, (kRecomputeUnits + bh - 1) / bh));
}

size_t bw_workspace_bytes(const dn_backward_args* a) {
  const int NC = (a->L + BC - 1) / BC, ncb = bw_block_chunks(a);
  const int nblk = (NC + ncb - 1) / ncb;
  const size_t bh = (size_t)a->B * a->H;
  // + the states at the nblk - 1 interior boundaries and one state gradient
  // carried between blocks
  const size_t extra = nblk > 1 ? (size_t)nblk * bh * KK : 0;
  return (bh * ncb * kUnitFloats + extra) * sizeof(float);
}

int bw_check(const dn_backward_args* a) {
  if (a == nullptr) return set_error(DN_E_INVALID, "null args");
  if (a->abi_version != DN_ABI_VERSION) return set_error(DN_E_ABI, "dn_backward_args built for another ABI version");
  if (a->K != KD || a->V != KD) return set_error(DN_E_INVALID, "K and V must both be 128");
  if (a->B <= 0 || a->L <= 0 || a->H <= 0) return set_error(DN_E_INVALID, "B, L and H must be positive");
  if (!a->q || !a->k || !a->v || !a->g || !a->b || !a->w || !a->d_out)
    return set_error(DN_E_INVALID, "missing input tensor pointer");
  if (!a->dq || !a->dk || !a->dv || !a->dg || !a->db || !a->dw)
    return set_error(DN_E_INVALID, "missing gradient tensor pointer");
  if (a->d_init != nullptr && a->init_state == nullptr)
    return set_error(DN_E_INVALID, "d_init needs init_state");
  return DN_OK;
}

}  // namespace

extern "C" size_t dn_prefill_bwd_workspace_size(const dn_backward_args* a) {
  if (bw_check(a) != DN_OK) return 0;
  return bw_workspace_bytes(a);
}

// the recurrence backward with the element types of d_out and dv given
static int bwd_core(const dn_backward_args* a, int dout_dt, int dv_dt, int v_dt, bool bf, void* workspace,
                    size_t workspace_bytes, void* stream, int qk_hd = 1, int gb_hd = 1) {
  const int rc = bw_check(a);
  if (rc != DN_OK) return rc;
  const size_t need = bw_workspace_bytes(a);
  if (workspace == nullptr || workspace_bytes < need) return set_error(DN_E_WORKSPACE, "workspace too small");
  const int NC = (a->L + BC - 1) / BC, ncb = bw_block_chunks(a);
  const int nblk = (NC + ncb - 1) / ncb;
  BW p{};
  p.B = a->B; p.L = a->L; p.H = a->H;
  p.bf = bf;
  p.q = (const float*)a->q; p.k = (const float*)a->k; p.v = (const float*)a->v;
  p.g = (const float*)a->g; p.b = (const float*)a->b; p.w = (const float*)a->w;
  p.qk_hd = qk_hd; p.gb_hd = gb_hd;
  p.seg = a->seg;
  p.dout = a->d_out; p.dout_dt = dout_dt; p.dv_dt = dv_dt; p.v_dt = v_dt;
  p.dq = (float*)a->dq; p.dk = (float*)a->dk; p.dv = (float*)a->dv;
  p.dg = (float*)a->dg; p.db = (float*)a->db; p.dw = (float*)a->dw;
  const size_t bh = (size_t)a->B * a->H;
  const size_t units = bh * ncb;   // per launch, at most
  float* ws = (float*)workspace;
  auto take = [&](size_t per) { float* r = ws; ws += units * per; return r; };
  p.G = take(CK); p.Wm = take(CK); p.WT = take(CK); p.Kc = take(CK); p.KcT = take(CK);
  p.PT = take(KK); p.U0T = take(CK); p.MT = take(CC); p.TT = take(CC); p.lam = take(KD);
  p.dMw = take(CC); p.dAw = take(CC); p.Rq = take(CK); p.Rk = take(CK); p.Rb = take(CK); p.RS = take(KD);
  p.S = take(KK); p.dS = take(KK);
  // the state entering block j (j >= 1), (B, H, K, V) each, then the carried
  // state gradient
  float* ckpt = ws;
  auto boundary = [&](int j) { return ckpt + (size_t)(j - 1) * bh * KK; };
  float* dcarry = nblk > 1 ? boundary(nblk) : nullptr;

  hipStream_t st = (hipStream_t)stream;
  // k_bw_intra is persistent: at most one workgroup per CU (its LDS allows one)
  int dev = 0, ncu = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      ncu <= 0)
    ncu = 256;
  auto intra_grid = [&](unsigned n) { return dim3(std::min(n, (unsigned)ncu)); };
  const int chains = a->B * a->H * chains_per_head(p.bf);
  auto chain_grid = [](int nb) { return dim3((unsigned)(8 * ((nb + 7) / 8))); };
  auto block = [&](int j) {
    p.c0 = j * ncb;
    p.NC = std::min(ncb, NC - p.c0);
    return (unsigned)(bh * p.NC);
  };
  prof_mark(4, st, false);
  // forward pass: the states at the block boundaries (the only states kept)
  for (int j = 0; j + 1 < nblk; ++j) {
    const unsigned n = block(j);
    p.init = j == 0 ? (const float*)a->init_state : boundary(j);
    p.sfin = boundary(j + 1);
    p.dfin = nullptr; p.dinit = nullptr;
    if (p.bf) hipLaunchKernelGGL(k_bw_intra<true>, intra_grid(n), dim3(NT), 0, st, p);
    else hipLaunchKernelGGL(k_bw_intra<false>, intra_grid(n), dim3(NT), 0, st, p);
    if (p.bf) hipLaunchKernelGGL(k_bw_chains<true>, chain_grid(chains), dim3(256), 0, st, p, chains, chains);
    else hipLaunchKernelGGL(k_bw_chains<false>, chain_grid(chains), dim3(256), 0, st, p, chains, chains);
  }
  // blocks from the last to the first: chunk products, both scans (the
  // forward one from the block's boundary state), gradients; the reverse
  // scan's state gradient at the block start carries into the block before
  // it (read and written in place by the same lanes)
  for (int j = nblk - 1; j >= 0; --j) {
    const unsigned n = block(j);
    p.init = j == 0 ? (const float*)a->init_state : boundary(j);
    p.sfin = nullptr;
    p.dfin = j == nblk - 1 ? (const float*)a->d_final : dcarry;
    p.dinit = j == 0 ? (float*)a->d_init : dcarry;
    if (p.bf) hipLaunchKernelGGL(k_bw_intra<true>, intra_grid(n), dim3(NT), 0, st, p);
    else hipLaunchKernelGGL(k_bw_intra<false>, intra_grid(n), dim3(NT), 0, st, p);
    if (p.bf) hipLaunchKernelGGL(k_bw_chains<true>, chain_grid(2 * chains), dim3(256), 0, st, p, chains, 2 * chains);
    else hipLaunchKernelGGL(k_bw_chains<false>, chain_grid(2 * chains), dim3(256), 0, st, p, chains, 2 * chains);
    if (p.bf) hipLaunchKernelGGL(k_bw_grads<true>, dim3(n), dim3(NT), 0, st, p);
    else hipLaunchKernelGGL(k_bw_grads<false>, dim3(n), dim3(NT), 0, st, p);
    hipLaunchKernelGGL(k_bw_dqk, dim3((unsigned)(NQ * n)), dim3(NT), 0, st, p);
  }
  prof_mark(4, st, true);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(DN_E_LAUNCH, hipGetErrorString(e));
  return DN_OK;
}

extern "C" int dn_prefill_bwd(const dn_backward_args* a, void* workspace, size_t workspace_bytes, void* stream) {
  return bwd_core(a, DT_F32, DT_F32, DT_F32, false, workspace, workspace_bytes, stream);
}

namespace {

// Prepared inputs and their gradients: qe, ke at the key heads; ge, be at
// Hv / gb_hd heads; ve, we and the five gradients at the value heads.
struct RawLayout {
  size_t canon, pre, pre_k, pre_gb, core;   // bytes (pre*: one array)
  int gb_hd;
  size_t total() const { return canon + 7 * pre + 2 * pre_k + 2 * pre_gb + core; }
};

RawLayout raw_layout(const dn_prefill_args* a) {
  RawLayout r;
  r.canon = (((size_t)a->B * a->L * sizeof(int32_t)) + 255) & ~(size_t)255;
  r.pre = (size_t)a->B * a->L * a->Hv * KD * sizeof(float);
  r.pre_k = (size_t)a->B * a->L * a->Hk * KD * sizeof(float);
  r.gb_hd = (a->g_heads == a->Hk && a->b_heads == a->Hk) ? a->Hv / a->Hk : 1;
  r.pre_gb = r.pre / r.gb_hd;
  dn_backward_args c{};
  c.B = a->B; c.L = a->L; c.H = a->Hv;
  c.recompute_states = a->recompute_states;
  r.core = bw_workspace_bytes(&c);
  return r;
}

int raw_check(const dn_prefill_args* a) {
  if (a == nullptr) return set_error(DN_E_INVALID, "null args");
  if (a->abi_version != DN_ABI_VERSION) return set_error(DN_E_ABI, "dn_prefill_args built for another ABI version");
  if (a->K != KD || a->V != KD) return set_error(DN_E_INVALID, "K and V must both be 128");
  if (a->B <= 0 || a->L <= 0 || a->Hk <= 0 || a->Hv <= 0 || a->Hv % a->Hk)
    return set_error(DN_E_INVALID, "bad batch / length / head counts");
  if (!a->q || !a->k || !a->v || !a->g || !a->b || !a->w) return set_error(DN_E_INVALID, "missing input tensor pointer");
  if (a->qk_dtype != DN_F32 && a->qk_dtype != DN_BF16 && a->qk_dtype != DN_F16)
    return set_error(DN_E_INVALID, "q/k dtype must be f32, bf16 or f16");
  if (a->v_dtype != DN_F32 && a->v_dtype != DN_BF16) return set_error(DN_E_INVALID, "v dtype must be f32 or bf16");
  const int hs[3] = {a->g_heads, a->b_heads, a->w_heads}, cs[3] = {a->g_chans, a->b_chans, a->w_chans};
  const int ds[3] = {a->g_dtype, a->b_dtype, a->w_dtype};
  for (int i = 0; i < 3; ++i) {
    if (ds[i] != DN_F32) return set_error(DN_E_INVALID, "gates must be f32");
    if (hs[i] != 1 && hs[i] != a->Hk && hs[i] != a->Hv) return set_error(DN_E_INVALID, "gate heads must be 1, Hk or Hv");
    if (cs[i] != 1 && cs[i] != KD) return set_error(DN_E_INVALID, "gate channels must be 1 or 128");
  }
  if (a->seg != nullptr && a->seg_dtype != DN_I32 && a->seg_dtype != DN_I64)
    return set_error(DN_E_INVALID, "segment ids must be i32 or i64");
  return DN_OK;
}

}  // namespace

extern "C" size_t dn_prefill_bwd_raw_workspace_size(const dn_prefill_args* a) {
  if (raw_check(a) != DN_OK) return 0;
  return raw_layout(a).total();
}

extern "C" int dn_prefill_bwd_raw(const dn_prefill_args* a, const void* d_out, const void* d_final,
                                  void* dq, void* dk, void* dv, void* dg, void* db, void* dw, void* d_init,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  int rc = raw_check(a);
  if (rc != DN_OK) return rc;
  if (!d_out || !dq || !dk || !dv || !dg || !db || !dw) return set_error(DN_E_INVALID, "missing gradient pointer");
  if (d_init != nullptr && a->init_state == nullptr) return set_error(DN_E_INVALID, "d_init needs init_state");
  const RawLayout lay = raw_layout(a);
  if (workspace == nullptr || workspace_bytes < lay.total())
    return set_error(DN_E_WORKSPACE, "workspace too small");
  char* w = (char*)workspace;
  BR r{};
  r.B = a->B; r.L = a->L; r.Hk = a->Hk; r.Hv = a->Hv; r.G = a->Hv / a->Hk;
  r.q = a->q; r.k = a->k; r.v = a->v; r.qk_dt = a->qk_dtype; r.v_dt = a->v_dtype;
  r.g = (const float*)a->g; r.b = (const float*)a->b; r.w = (const float*)a->w;
  r.g_h = a->g_heads; r.g_c = a->g_chans; r.b_h = a->b_heads; r.b_c = a->b_chans; r.w_h = a->w_heads; r.w_c = a->w_chans;
  r.seg = a->seg; r.seg_dt = a->seg_dtype; r.seg_batched = a->seg_batched;
  r.init_seg = a->init_seg; r.has_init = a->init_state != nullptr;
  r.scale = a->scale; r.l2norm = a->qk_l2norm; r.fuse = a->fuse_prologue; r.guard = a->stability_guard;
  r.canon = (int32_t*)w; w += lay.canon;
  float* pre[11];
  for (int i = 0; i < 11; ++i) {
    pre[i] = (float*)w;
    w += i < 2 ? lay.pre_k : (i == 3 || i == 4) ? lay.pre_gb : lay.pre;
  }
  r.qe = pre[0]; r.ke = pre[1]; r.ve = pre[2]; r.ge = pre[3]; r.be = pre[4]; r.we = pre[5];
  r.dqe = pre[6]; r.dke = pre[7]; r.dge = pre[8]; r.dbe = pre[9]; r.dwe = pre[10];
  // the recurrence kernels read w in place when its prologue step is the
  // identity on a per-value-head, channel-wise layout
  r.w_alias = !a->fuse_prologue && !a->stability_guard && a->w_heads == a->Hv && a->w_chans == KD;
  r.gb_hd = lay.gb_hd;
  r.dq = (float*)dq; r.dk = (float*)dk; r.dg = (float*)dg; r.db = (float*)db; r.dw = (float*)dw;

  hipStream_t st = (hipStream_t)stream;
  const int64_t rows = (int64_t)a->B * a->L * a->Hv;
  hipLaunchKernelGGL(k_bw_prep, dim3((unsigned)((rows + 7) / 8 + a->B)), dim3(256), 0, st, r);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(DN_E_LAUNCH, hipGetErrorString(e));

  dn_backward_args c{};
  c.abi_version = DN_ABI_VERSION;
  c.B = a->B; c.L = a->L; c.H = a->Hv; c.K = KD; c.V = KD;
  c.q = r.qe; c.k = r.ke; c.v = r.ve; c.g = r.ge; c.b = r.be; c.w = r.w_alias ? a->w : r.we;
  c.seg = r.canon; c.init_state = a->init_state; c.d_out = d_out; c.d_final = d_final;
  // without the fused prologue, w's step has derivative 1: at Hv heads and
  // channel-wise the recurrence backward writes dw in its raw layout itself
  const bool dw_direct = !a->fuse_prologue && a->w_heads == a->Hv && a->w_chans == KD;
  c.dq = pre[6]; c.dk = pre[7]; c.dv = dv; c.dg = pre[8]; c.db = pre[9]; c.dw = dw_direct ? (float*)dw : pre[10];
  c.d_init = d_init;
  c.recompute_states = a->recompute_states;
  rc = bwd_core(&c, a->v_dtype, a->v_dtype, DT_F32, a->precision == 0, w, lay.core, stream, a->Hv / a->Hk, r.gb_hd);
  if (rc != DN_OK) return rc;

  const int64_t krows = (int64_t)a->B * a->L * a->Hk;
  const int64_t ng = (int64_t)a->B * a->L * a->g_heads * a->g_chans;
  const int64_t nb = (int64_t)a->B * a->L * a->b_heads * a->b_chans;
  const int64_t nw = (int64_t)a->B * a->L * a->w_heads * a->w_chans;
  // channel-wise gates take the float4 kernels (8 rows of 128 channels per
  // block); at the key heads they share the dq / dk launch
  const bool gb4 = a->g_chans == KD && a->b_chans == KD && a->g_heads == a->b_heads;
  if (gb4 && a->g_heads == a->Hk) {
    hipLaunchKernelGGL(k_bw_post_qkgb, dim3((unsigned)((krows + 7) / 8)), dim3(256), 0, st, r);
  } else if (gb4) {
    hipLaunchKernelGGL(k_bw_post_qk, dim3((unsigned)((krows + 7) / 8)), dim3(256), 0, st, r);
    hipLaunchKernelGGL(k_bw_post_gate4_gb, dim3((unsigned)((ng / KD + 7) / 8)), dim3(256), 0, st, r);
  } else {
    hipLaunchKernelGGL(k_bw_post_qk, dim3((unsigned)((krows + 7) / 8)), dim3(256), 0, st, r);
    if (a->g_chans == KD) hipLaunchKernelGGL(k_bw_post_gate4<0>, dim3((unsigned)((ng / KD + 7) / 8)), dim3(256), 0, st, r);
    else hipLaunchKernelGGL(k_bw_post_gate<0>, dim3((unsigned)((ng + 255) / 256)), dim3(256), 0, st, r);
    if (a->b_chans == KD) hipLaunchKernelGGL(k_bw_post_gate4<1>, dim3((unsigned)((nb / KD + 7) / 8)), dim3(256), 0, st, r);
    else hipLaunchKernelGGL(k_bw_post_gate<1>, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, st, r);
  }
  if (!dw_direct) {
    if (a->w_chans == KD) hipLaunchKernelGGL(k_bw_post_gate4<2>, dim3((unsigned)((nw / KD + 7) / 8)), dim3(256), 0, st, r);
    else hipLaunchKernelGGL(k_bw_post_gate<2>, dim3((unsigned)((nw + 255) / 256)), dim3(256), 0, st, r);
  }
  e = hipGetLastError();
  if (e != hipSuccess) return set_error(DN_E_LAUNCH, hipGetErrorString(e));
  return DN_OK;
}
