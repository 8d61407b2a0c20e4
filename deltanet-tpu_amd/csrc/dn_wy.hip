// Chunk-parallel prefill for precision="bf16" on gfx950: four launches per
// token block instead of one workgroup doing every product of a chunk.
//
// Reference algorithm (maelie-labs/deltanet-tpu v0.3.0, src/deltanet_tpu/):
//   prepass   gdn2.py:115-240   (Lambda, A, M, T = (I+A)^-1, W, U, qe, ke)
//   state     gdn2.py:585-652   (Vnew = U - W S, O = qe S + M Vnew,
//                                S <- [same doc] diag(e^Lend) S + ke^T Vnew)
//   flags     gdn2.py:1291-1302, wrapper gdn2.py:1970-2125
//
// With W = T be and U = T wv (be = b k e^Lambda, wv = w v) the per-chunk map
// is affine in the state, and every operator in it factors through
//     R = [R_O; R_Q] = [M; ke^T] T                       (256 x 128)
// as
//     X  = qe - R_O be,  Oi = R_O wv      (output  O = X S + Oi)
//     Pn = -R_Q be,      Q  = R_Q wv      (state   S' = [same] D S + Pn S + Q)
// so the work splits into
//   k_wy   one 8-wave workgroup per (batch, exec head, chunk): chunk flags,
//          Lambda, A and M (MFMA on exp-scaled operands), T by blocked
//          inversion, R, and the transposed be / qe the next launch needs;
//   k_val  four workgroups per unit: R [-be | wv] (X, Pn, Oi, Q);
//   k_scan one workgroup per (batch, exec head, 16 state columns): the
//          sequential recurrence, storing every chunk's entering state;
//   k_out  chunk-parallel output O^T = S_c^T X^T + Oi^T.
// Every intermediate is stored in the MFMA lane order of its consumer
// ("fragment-native", fofs / cofs in dn_common.h).
//
// Decay factors (all in registers or LDS, never as extra HBM passes):
//   scalar decay (one g per token and head): A and M are products of the raw
//     operands scaled per element by e^{Lambda_i - Lambda_j};
//   per-channel decay, spans within 2^{+-99} of row 64 ("midpoint"): every
//     entry factors as (row: e^{Lambda_i - Lambda_64}) (col: e^{Lambda_64 -
//     Lambda_j}), so A and M are single products over all 128 tokens;
//   otherwise ("blockwise"): row factors relative to the row's 16-token block,
//     column factors rescaled per block pair by e^{Lambda_a0 - Lambda_c15}
//     (every factor <= 1), and 16-token diagonal blocks whose own span
//     exceeds 2^99 summed per element.
// Every exponent is a sum of gates of one sign, formed from block-local
// partial sums, so no factor is a difference of two large cumulative sums.
#include "dn_common.h"
#include "dn_host.h"

namespace dn {
namespace wy {

constexpr int CH = 128;
constexpr int KD = 128;
constexpr int TP = 132;                 // fp32 LDS pitch (floats) of A^T / T^T
constexpr float kSafeNat = 68.6f;       // e^{68.6} < 2^{99}
constexpr int SQ = CH * KD;             // elements of one 128 x 128 operand

#ifdef DN_STAMPS
// phase timestamps of one workgroup per launch (probe builds only)
__device__ unsigned long long dn_stamp_buf[8][64];
#define DN_STAMP(kern, k)                                                             \
  do {                                                                                \
    if (blockIdx.x == DN_STAMPS && threadIdx.x < 64)                                  \
      dn_stamp_buf[kern][(k) + 32 * (threadIdx.x >> 5) * 0] = __builtin_amdgcn_s_memtime(); \
  } while (0)
#define DN_RSTAMP(kern, k)                                                            \
  do {                                                                                \
    if (blockIdx.x == DN_STAMPS && threadIdx.x < 64) dn_stamp_buf[kern][k] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#else
#define DN_STAMP(kern, k) do {} while (0)
#define DN_RSTAMP(kern, k) do {} while (0)
#endif
__device__ __forceinline__ float sigmoid_fast(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }
__device__ __forceinline__ float expn(float x) { return fast_exp2(x * kLog2e); }

// inclusive prefix sum over the 16 lanes of a DPP row (lanes 16q .. 16q+15)
__device__ __forceinline__ float row_scan16(float x) {
#define DN_DPP_ADD(ctrl) x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), ctrl, 0xf, 0xf, true))
  DN_DPP_ADD(0x111);
  DN_DPP_ADD(0x112);
  DN_DPP_ADD(0x114);
  DN_DPP_ADD(0x118);
#undef DN_DPP_ADD
  return x;
}
// inclusive suffix sum over the 16 lanes of a DPP row
__device__ __forceinline__ float row_rscan16(float x) {
#define DN_DPP_ADD(ctrl) x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), ctrl, 0xf, 0xf, true))
  DN_DPP_ADD(0x101);
  DN_DPP_ADD(0x102);
  DN_DPP_ADD(0x104);
  DN_DPP_ADD(0x108);
#undef DN_DPP_ADD
  return x;
}
// value of the next lane in the DPP row (0 in the row's last lane)
__device__ __forceinline__ float row_next(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x101, 0xf, 0xf, true));
}

__device__ __forceinline__ int kgate_head(const PF& p, int H, int h) {
  if (H == 1) return 0;
  if (p.gates_at_hv) return (H == p.Hv) ? h : h / p.G;
  return h;
}
__device__ __forceinline__ int vgate_head(const PF& p, int H, int hv) {
  if (H == 1) return 0;
  return (H == p.Hv) ? hv : hv / p.G;
}

struct SegId {
  int32_t lo, hi;
  __device__ __forceinline__ bool operator!=(const SegId& o) const { return lo != o.lo || hi != o.hi; }
};
__device__ __forceinline__ SegId seg_raw(const PF& p, int b, int t) {
  const int64_t i = p.seg_batched ? (int64_t)b * p.L + t : (int64_t)t;
  const bool w64 = p.seg_dt == DT_I64;
  const int32_t* s32 = (const int32_t*)p.seg + (w64 ? 2 * i : i);
  const int32_t hi = s32[w64 ? 1 : 0];
  return SegId{s32[0], w64 ? hi : 0};
}

using P = Pol<true>;
using F1 = P::F1;
using F3 = P::F3;
using SS = Store<true>;

// split fragment (hi, lo) of a 128 x 128 fragment-native bf16 pair of arrays
__device__ __forceinline__ F3 ldf3(const bf16* base, int tile, int slab, int l) {
  const int o = fofs(tile, slab, l);
  return SS::fa3(base + o, base + SQ + o);
}
__device__ __forceinline__ void stf3(bf16* base, int tile, int slab, int l, const float* x) {
  const int o = fofs(tile, slab, l);
  SS::st8s(base + o, base + SQ + o, x);
}
// 8 fp32 values of a fragment-native fp32 array
__device__ __forceinline__ void ld8f(const float* base, int tile, int slab, int l, float* x) {
  const int o = fofs(tile, slab, l);
  const f32x4 a = *reinterpret_cast<const f32x4*>(base + o);
  const f32x4 b = *reinterpret_cast<const f32x4*>(base + o + 4);
#pragma unroll
  for (int e = 0; e < 4; ++e) { x[e] = a[e]; x[4 + e] = b[e]; }
}
// x[e] = rowp[pi(q, e)] from a row-major fp32 row at the slab start
__device__ __forceinline__ void row8f(const float* rowp, int q, float* x) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(rowp + 4 * q);
  const f32x4 b = *reinterpret_cast<const f32x4*>(rowp + 16 + 4 * q);
#pragma unroll
  for (int e = 0; e < 4; ++e) { x[e] = a[e]; x[4 + e] = b[e]; }
}

// The transposed halves of a row fragment: an exact product with the two
// halves of a 32 x 32 identity.  Returns, in accumulator layout, lane
// (n, q) = value (row 4q + ii, column 16 half + n) of the 16 x 32 fragment.
__device__ __forceinline__ f32x4 tr_half(const F1& a, int half, int r16, int q) {
  f32x4 c = zero4();
  mma(c, a, ident_frag<true>(half, r16, q));
  return c;
}

// ===========================================================================
// k_wy: chunk operators.  Wave w owns token block w (rows 16w .. 16w+15) for
// the per-token work; the A and M tile products are balanced as nine tiles
// per wave: A tiles (w, c <= w) and M^T tiles (c, 7-w), c < 7-w, plus the
// diagonal M^T tile (w, w).
//
// LDS: smP  C operand (split, midpoint / scalar) or k e^{tail} (fp32,
//           blockwise), then A^T and T^T (fp32, pitch 132);
//      smQ  block table, then the row operand of M (split), then ke^T
//           fragments (split);
//      smT  per-channel factor tables, then the T scratch.
// ===========================================================================
template <class TIn, class TV>
__global__ __launch_bounds__(512) void k_wy(const PF p) {
  __shared__ __align__(16) float smP[CH * TP];
  __shared__ __align__(16) bf16 smQ[2 * SQ];
  __shared__ __align__(16) float smT[6656];
  __shared__ int doc[CH];
  __shared__ int misc[16];
  __shared__ float tokv[4 * CH];   // scalar decay: per-token loc, tail, e^Lambda, e^{Lend - Lambda}

  DN_STAMP(0, 0);
  DN_RSTAMP(0, 16);
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l = tid & 63, r16 = l & 15, q = l >> 4;
  const int units = p.B * p.Hx * p.NCb;
  int c, h, b;
  {
    int id = blockIdx.x;
    if ((units & 7) == 0) id = (id & 7) * (units >> 3) + (id >> 3);
    c = id % p.NCb;
    id /= p.NCb;
    h = id % p.Hx;
    b = id / p.Hx;
  }
  const int tb = p.t0 + c * CH;
  const int t_end = min(p.t0 + p.nt, p.L);
  const int64_t u = ((int64_t)b * p.Hx + h) * p.NCb + c;
  const int hk = p.gates_at_hv ? h / p.G : h;
  const bool scalar_g = p.g_c == 1;

  // ---- entry loads: segment ids, then the rows of token block w ----------
  SegId sg_t{0, 0}, sg_tp{0, 0}, sg_0{0, 0}, sg_a{0, 0}, sg_b{0, 0};
  int32_t iseg = 0;
  if (p.seg != nullptr) {
    const int ti = tid & (CH - 1);
    sg_t = seg_raw(p, b, min(tb + ti, t_end - 1));
    sg_tp = seg_raw(p, b, max(min(tb + ti - 1, t_end - 1), 0));
    sg_0 = seg_raw(p, b, 0);
    sg_a = seg_raw(p, b, tb);
    sg_b = seg_raw(p, b, max(tb - 1, 0));
  }
  if (p.init_seg != nullptr) iseg = p.init_seg[b];
  // rows of token block `blk` (this lane: token 16 blk + r16)
  struct Rows {
    Raw8<TIn> q[4], k[4];
    Raw8<float> b[4], g[4];
    float b_sc, g_sc;
  };
  auto load_rows = [&](int blk, Rows& R) {
    const int ti = 16 * blk + r16;
    const bool ok = tb + ti < t_end;
    const int64_t bt = (int64_t)b * p.L + (ok ? tb + ti : tb);
    const int hg = kgate_head(p, p.g_h, h), hb = kgate_head(p, p.b_h, h);
    const float* gp = (const float*)p.g + (bt * p.g_h + hg) * p.g_c;
    const float* bp = (const float*)p.b + (bt * p.b_h + hb) * p.b_c;
    R.g_sc = 0.f;
    R.b_sc = 0.f;
    if (scalar_g) {
      R.g_sc = gp[0];
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) R.g[s].load(gp + 32 * s, q);
    }
    const TIn* qp = (const TIn*)p.q + (bt * p.Hk + hk) * KD;
    const TIn* kp = (const TIn*)p.k + (bt * p.Hk + hk) * KD;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      R.q[s].load(qp + 32 * s, q);
      R.k[s].load(kp + 32 * s, q);
    }
    if (p.b_c == 1) {
      R.b_sc = bp[0];
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) R.b[s].load(bp + 32 * s, q);
    }
  };
  const int i_row = 16 * w + r16;             // this lane's token in the chunk
  const bool valid = tb + i_row < t_end;
  Rows rw;
  load_rows(w, rw);
  asm volatile("" : "+v"(sg_t.lo), "+v"(sg_t.hi), "+v"(sg_tp.lo), "+v"(sg_tp.hi));
  asm volatile("" : "+v"(sg_0.lo), "+v"(sg_0.hi), "+v"(sg_a.lo), "+v"(sg_a.hi), "+v"(sg_b.lo), "+v"(sg_b.hi));

  DN_STAMP(0, 1);
  // ---- phase 0: in-chunk document index, chunk flags ----------------------
  if (w < 2) {
    const bool chg = (p.seg != nullptr && tid > 0) ? (sg_t != sg_tp) : false;
    const uint64_t bal = __ballot(chg);
    doc[tid] = __popcll(bal & (l == 63 ? ~0ull : ((2ull << l) - 1)));
    if (w == 0 && l == 0) misc[0] = __popcll(bal);
  }
  lds_barrier();
  if (w == 1) doc[tid] += misc[0];
  if (tid == 0 && h == 0) {
    int is_new;
    if (tb == 0) {
      if (p.has_init) {
        is_new = 0;
        if (p.init_seg != nullptr)
          is_new = (sg_0.lo != iseg) || (p.seg_dt == DT_I64 && sg_0.hi != (iseg < 0 ? -1 : 0));
      } else {
        is_new = 1;
      }
    } else if (c == 0 && !p.has_init) {
      is_new = 1;
    } else {
      is_new = p.seg ? (sg_a != sg_b) : 0;
    }
    p.flags[((int64_t)b * p.NCb + c) * 2 + 0] = is_new;
  }

  DN_STAMP(0, 2);
  // ---- phase 1: gates, block-local decay sums ------------------------------
  // loc = sum of g over tokens (16w, i] of the row's block (<= 0), tl = sum
  // over (i, 16w+15]; the block total (tokens 16w+1 .. 16w+15) and the
  // block's first gate go to a table.
  float* tbl = reinterpret_cast<float*>(smQ);   // [2][8][128]: totals, first gates
  const float gmax = p.guard ? -1e-6f : 0.f;
  auto act_g = [&](float x, bool ok) {
    x = p.fuse ? -__expf(fminf(x, 5.f)) : fminf(x, 0.f);   // fminf(NaN, 0) = 0
    return ok ? fminf(x, gmax) : 0.f;
  };
  float loc[32], gv[32];
  if (scalar_g) {
    const float gs = act_g(rw.g_sc, valid);
    const float ls = row_scan16(r16 == 0 ? 0.f : gs);
    if (q == 0) tokv[i_row] = ls;
    if (l == 15) tbl[w] = ls;
    if (l == 0) tbl[8 + w] = gs;
  } else {
#pragma unroll
    for (int s = 0; s < 4; ++s) rw.g[s].to(gv + 8 * s);
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      gv[e] = act_g(gv[e], valid);
      loc[e] = row_scan16(r16 == 0 ? 0.f : gv[e]);
    }
    if (r16 == 15) {
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int e = 0; e < 8; ++e) tbl[w * KD + 32 * s + pi_k(q, e)] = loc[8 * s + e];
    }
    if (r16 == 0) {
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int e = 0; e < 8; ++e) tbl[8 * KD + w * KD + 32 * s + pi_k(q, e)] = gv[8 * s + e];
    }
  }
  lds_barrier();
  if (tid == 0 && h == 0) p.flags[((int64_t)b * p.NCb + c) * 2 + 1] = (doc[CH - 1] == 0);

  DN_STAMP(0, 3);
  // ---- phase 2: per-channel (or per-token) factor tables -------------------
  // smT.  midpoint: off[8][128] (Lambda_16a - Lambda_64), eL64[128], eE64[128];
  // blockwise: F[28][128], eLa[8][128], eEa[8][128], kdf[8][128];
  // scalar: per-token e^Lambda, e^{Lend - Lambda} in tokv, pair sums D[28].
  float* t_off = smT;             // midpoint
  float* t_eL64 = smT + 8 * KD;
  float* t_eE64 = smT + 9 * KD;
  float* t_F = smT;               // blockwise
  float* t_eLa = smT + 28 * KD;
  float* t_eEa = smT + 36 * KD;
  float* t_kdf = smT + 44 * KD;
  float* dvec = p.dvec + u * KD;
  bool midpoint = false;
  if (scalar_g) {
    if (tid < CH) {
      const int i = tid, a = i >> 4;
      float pre = 0.f;   // Lambda at the first token of block a
      for (int bb = 0; bb < a; ++bb) pre += tbl[8 + bb] + tbl[bb];
      pre += tbl[8 + a];
      float post = 0.f;  // sum over the blocks after a
      for (int bb = a + 1; bb < 8; ++bb) post += tbl[8 + bb] + tbl[bb];
      const float li = tokv[i];
      const float tail = tbl[a] - li;
      tokv[2 * CH + i] = expn(pre + li);         // e^{Lambda_i}
      tokv[3 * CH + i] = expn(tail + post);      // e^{Lambda_end - Lambda_i}
      tokv[CH + i] = tail;
      if (i == CH - 1) {
        float all = 0.f;
        for (int bb = 0; bb < 8; ++bb) all += tbl[8 + bb] + tbl[bb];
        misc[4] = __float_as_int(expn(all));
      }
    } else if (tid < CH + 28) {
      // D(a, c) = sum of g over (16c+15, 16a], c < a
      const int pr = tid - CH;
      int a = 1;
      while (a * (a + 1) / 2 <= pr) ++a;
      const int cc = pr - a * (a - 1) / 2;
      float sm = 0.f;
      for (int bb = cc + 1; bb < a; ++bb) sm += tbl[8 + bb] + tbl[bb];
      sm += tbl[8 + a];
      smT[pr] = sm;
    }
    lds_barrier();
    if (tid < KD) dvec[tid] = __int_as_float(misc[4]);
  } else {
    if (tid < KD) {
      const int r = tid;
      float tot[8], fst[8];
#pragma unroll
      for (int a = 0; a < 8; ++a) { tot[a] = tbl[a * KD + r]; fst[a] = tbl[8 * KD + a * KD + r]; }
      // lo[a] = sum over (16a, 64] (a < 4); hi[a] = sum over (64, 16a] (a > 4)
      float lo[4], hi[8];
      float acc = fst[4];
#pragma unroll
      for (int a = 3; a >= 0; --a) { acc += tot[a]; lo[a] = acc; acc += fst[a]; }
      const float lam64 = acc;   // sum over [0, 64]
      float acc2 = tot[4];
#pragma unroll
      for (int a = 5; a < 8; ++a) { acc2 += fst[a]; hi[a] = acc2; acc2 += tot[a]; }
      // acc2 = sum over (64, 127]
#pragma unroll
      for (int a = 0; a < 4; ++a) t_off[a * KD + r] = -lo[a];
      t_off[4 * KD + r] = 0.f;
#pragma unroll
      for (int a = 5; a < 8; ++a) t_off[a * KD + r] = hi[a];
      t_eL64[r] = expn(lam64);
      t_eE64[r] = expn(acc2);
      dvec[r] = expn(lam64 + acc2);
      const bool unsafe = (-lo[0] > kSafeNat) || (-acc2 > kSafeNat);
      const bool any_unsafe = __any(unsafe);
      if (l == 0) misc[2 + w] = any_unsafe;
    }
    lds_barrier();
    midpoint = __builtin_amdgcn_readfirstlane(!(misc[2] | misc[3]));
    if (!midpoint) {
      if (tid < KD) {
        const int r = tid;
        float tot[8], fst[8];
#pragma unroll
        for (int a = 0; a < 8; ++a) { tot[a] = tbl[a * KD + r]; fst[a] = tbl[8 * KD + a * KD + r]; }
        float pre = 0.f;
#pragma unroll
        for (int a = 0; a < 8; ++a) {
          t_eLa[a * KD + r] = expn(pre + fst[a]);   // e^{Lambda_16a}
          pre += fst[a] + tot[a];
        }
        float post = 0.f;
#pragma unroll
        for (int a = 7; a >= 0; --a) {
          t_eEa[a * KD + r] = expn(post);          // e^{Lambda_end - Lambda_{16a+15}}
          post += fst[a] + tot[a];
        }
        int bits = 0;
#pragma unroll
        for (int a = 0; a < 8; ++a) {
          t_kdf[a * KD + r] = expn(-tot[a]);
          bits |= (__any(-tot[a] > kSafeNat) ? 1 : 0) << a;
        }
#pragma unroll
        for (int a = 1; a < 8; ++a) {
          float sm = 0.f;
#pragma unroll
          for (int cc = a - 1; cc >= 0; --cc) {
            // F(a, cc) = e^{sum over (16cc+15, 16a]}
            sm += (cc == a - 1) ? fst[a] : (fst[cc + 1] + tot[cc + 1]);
            t_F[(a * (a - 1) / 2 + cc) * KD + r] = expn(sm);
          }
        }
        if (l == 0) misc[6 + w] = bits;
      }
      lds_barrier();
    }
  }
  const int diag_bad = (midpoint || scalar_g) ? 0 : __builtin_amdgcn_readfirstlane(misc[6] | misc[7]);

  DN_STAMP(0, 4);
  // ---- phase 3: q / k normalisation (gdn2.py:2113-2122: the normalised q, k
  // are stored back in the input dtype; the fused prologue, gdn2.py:133-142,
  // keeps them in fp32) --------------------------------------------------------
  auto norms = [&](const Rows& R, float& nq, float& nk) {
    float ssq = 0.f, ssk = 0.f;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      float xq[8], xk[8];
      R.q[s].to(xq);
      R.k[s].to(xk);
#pragma unroll
      for (int e = 0; e < 8; ++e) { ssq += xq[e] * xq[e]; ssk += xk[e] * xk[e]; }
    }
    ssq += __shfl_xor(ssq, 16); ssq += __shfl_xor(ssq, 32);
    ssk += __shfl_xor(ssk, 16); ssk += __shfl_xor(ssk, 32);
    nq = rsqrtf(ssq + 1e-6f);
    nk = rsqrtf(ssk + 1e-6f);
  };
  // prepared q, k and b * k of slab s
  auto prep = [&](const Rows& R, int s, float nq, float nk, bool ok, float* qv, float* kv, float* bk) {
    R.q[s].to(qv);
    R.k[s].to(kv);
    if (p.b_c == 1) {
#pragma unroll
      for (int e = 0; e < 8; ++e) bk[e] = R.b_sc;
    } else {
      R.b[s].to(bk);
    }
    if (p.fuse) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        qv[e] = (qv[e] * nq) * p.scale;
        kv[e] = kv[e] * nk;
        bk[e] = sigmoid_fast(bk[e]);
      }
    } else if (p.l2norm) {
#pragma unroll
      for (int e = 0; e < 8; ++e) { qv[e] = round_as<TIn>((qv[e] * nq) * p.scale); kv[e] = round_as<TIn>(kv[e] * nk); }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) qv[e] = round_as<TIn>(qv[e] * p.scale);
    }
    if (p.guard && !p.fuse) {
#pragma unroll
      for (int e = 0; e < 8; ++e) bk[e] = fmaxf(bk[e], 0.f);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      qv[e] = ok ? qv[e] : 0.f;
      kv[e] = ok ? kv[e] : 0.f;
      bk[e] = ok ? bk[e] * kv[e] : 0.f;
    }
  };
  float nq, nk;
  norms(rw, nq, nk);
  const bool first_doc = doc[i_row] == 0;
  const bool last_doc = doc[i_row] == doc[CH - 1];

  DN_STAMP(0, 5);
  // ---- phase 4: operands, one 32-channel slab at a time ---------------------
  // rowA: row operand of A (registers); row operand of M -> smQ (split);
  // column operand -> smP (split; fp32 k e^{tail} when blockwise);
  // kdF: blockwise diagonal column operand k e^{-loc} (registers).
  // be^T and ke^T fragments (identity transposes) and qe (accumulator layout
  // of X^T) go to the workspace.
  bf16* smQb = smQ;
  bf16* smPb = reinterpret_cast<bf16*>(smP);
  float* smPf = smP;
  bf16* gBe = (bf16*)p.BeF + u * SQ;
  float* gQe = p.QeC + u * SQ;
  F3 rowA[4], kdF[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    float qv[8], kv[8], bk[8];
    prep(rw, s, nq, nk, valid, qv, kv, bk);
    float ra[8], rm[8], be[8], qe[8];
    if (scalar_g) {
      const float eL = tokv[2 * CH + i_row];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        ra[e] = bk[e];
        rm[e] = qv[e];
        be[e] = bk[e] * eL;
        qe[e] = qv[e] * eL;
      }
      stf3(smPb, w, s, l, kv);
    } else if (midpoint) {
      float off[8], eL[8], cc[8];
      row8f(t_off + w * KD + 32 * s, q, off);
      row8f(t_eL64 + 32 * s, q, eL);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float E = expn(loc[8 * s + e] + off[e]);   // e^{Lambda_i - Lambda_64}
        ra[e] = bk[e] * E;
        rm[e] = qv[e] * E;
        cc[e] = kv[e] * __builtin_amdgcn_rcpf(E);
        be[e] = ra[e] * eL[e];
        qe[e] = rm[e] * eL[e];
      }
      stf3(smPb, w, s, l, cc);
    } else {
      float eL[8], kf[8], kc[8], kd[8];
      row8f(t_eLa + w * KD + 32 * s, q, eL);
      row8f(t_kdf + w * KD + 32 * s, q, kf);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float E = expn(loc[8 * s + e]);            // e^{Lambda_i - Lambda_16w}
        ra[e] = bk[e] * E;
        rm[e] = qv[e] * E;
        const float tl = row_next(row_rscan16(gv[8 * s + e]));   // sum over (i, 16w+15]
        kc[e] = kv[e] * expn(tl);                        // e^{Lambda_{16w+15} - Lambda_i}
        kd[e] = kc[e] * kf[e];
        be[e] = ra[e] * eL[e];
        qe[e] = rm[e] * eL[e];
      }
      kdF[s] = P::f3(kd);
      const int o = fofs(w, s, l);
      *reinterpret_cast<f32x4*>(smPf + o) = f32x4{kc[0], kc[1], kc[2], kc[3]};
      *reinterpret_cast<f32x4*>(smPf + o + 4) = f32x4{kc[4], kc[5], kc[6], kc[7]};
    }
    rowA[s] = P::f3(ra);
    stf3(smQb, w, s, l, rm);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      be[e] = first_doc ? be[e] : 0.f;
      qe[e] = first_doc ? qe[e] : 0.f;
    }
    const F1 fb = P::f1(be);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int o = fofs(2 * s + hf, w >> 1, l) + 4 * (w & 1);
      const f32x4 cb = tr_half(fb, hf, r16, q);
      const float xb[4] = {cb[0], cb[1], cb[2], cb[3]};
      SS::st4(gBe + o, xb);
      *reinterpret_cast<f32x4*>(gQe + cofs(2 * s + hf, w, 8, l)) =
          f32x4{qe[4 * hf], qe[4 * hf + 1], qe[4 * hf + 2], qe[4 * hf + 3]};
    }
  }
  lds_barrier();

  DN_STAMP(0, 6);
  // ---- phase 5: A and M^T tiles ----------------------------------------------
  // At[cc]: A tile (w, cc), lane (j, q) = A[16w + 4q + ii][16cc + j], cc <= w.
  // M^T tiles (cc, am), cc < am, lane (i, q) = M[16am + i][16cc + 4q + ii], are
  // masked and stored as they are formed; Md = M^T tile (w, w) waits for the
  // per-element diagonal blocks.
  const int am = 7 - w;
  bf16* gM = (bf16*)p.MF + u * 2 * SQ;
  f32x4 At[8], Md = zero4();
#pragma unroll
  for (int x = 0; x < 8; ++x) At[x] = zero4();
  // e^{Lambda_i - Lambda_j} for scalar decay (<= 1 wherever kept)
  auto dec = [&](int i, int j) {
    const int ai = i >> 4, cj = j >> 4;
    const float ex = (ai == cj) ? fminf(tokv[i] - tokv[j], 0.f) : tokv[i] + smT[ai * (ai - 1) / 2 + cj] + tokv[CH + j];
    return expn(ex);
  };
  auto store_mt = [&](int cc, f32x4 m) {
    const int i = 16 * am + r16;
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const int j = 16 * cc + 4 * q + ii;
      if (scalar_g) m[ii] *= dec(i, j);
      if (doc[i] != doc[j]) m[ii] = 0.f;
    }
    const float x[4] = {m[0], m[1], m[2], m[3]};
    const int o = fofs(am, cc >> 1, l) + 4 * (cc & 1);
    SS::st4s(gM + o, gM + SQ + o, x);
  };
  if (midpoint || scalar_g) {
    // every column-operand fragment is read from LDS once and serves both
    // the A tile (w, cc) and the M^T tile (cc, am)
    F3 rq[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) rq[s] = ldf3(smQb, am, s, l);
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) {
      if (cc <= w || cc < am) {
        F3 cf[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) cf[s] = ldf3(smPb, cc, s, l);
        if (cc <= w) {
#pragma unroll
          for (int s = 0; s < 4; ++s) P::m33(At[cc], rowA[s], cf[s]);
        }
        if (cc < am) {
          f32x4 m = zero4();
#pragma unroll
          for (int s = 0; s < 4; ++s) P::m33(m, cf[s], rq[s]);
          store_mt(cc, m);
        }
        if (cc == w) {
#pragma unroll
          for (int s = 0; s < 4; ++s) P::m33(Md, cf[s], ldf3(smQb, w, s, l));
        }
      }
    }
    if (scalar_g) {
#pragma unroll
      for (int cc = 0; cc < 8; ++cc) {
        if (cc <= w) {
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) At[cc][ii] *= dec(16 * w + 4 * q + ii, 16 * cc + r16);
        }
      }
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) Md[ii] *= dec(16 * w + r16, 16 * w + 4 * q + ii);
    }
  } else {
    // blockwise: column operand of pair (a, cc) = (k e^{tail})_cc * F(a, cc)
    auto colop = [&](int a, int cc, int s) -> F3 {
      float x[8], f[8];
      ld8f(smPf, cc, s, l, x);
      row8f(t_F + (a * (a - 1) / 2 + cc) * KD + 32 * s, q, f);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] *= f[e];
      return P::f3(x);
    };
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) {
      if (cc < w) {
#pragma unroll
        for (int s = 0; s < 4; ++s) P::m33(At[cc], rowA[s], colop(w, cc, s));
      }
      if (cc < am) {
        f32x4 m = zero4();
#pragma unroll
        for (int s = 0; s < 4; ++s) P::m33(m, colop(am, cc, s), ldf3(smQb, am, s, l));
        store_mt(cc, m);
      }
    }
    if (!((diag_bad >> w) & 1)) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        P::m33(At[w], rowA[s], kdF[s]);
        P::m33(Md, kdF[s], ldf3(smQb, w, s, l));
      }
    }
  }
  lds_barrier();

  // ke = k e^{Lend - Lambda} (last document) from the column operand still in
  // smP, transposed to ke^T fragments (rows = key channel, k = token) in smQ,
  // which the A / M products no longer read
  {
    const bool lastd = last_doc;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      float x[8], f[8];
      if (!midpoint && !scalar_g) {
        ld8f(smPf, w, s, l, x);                      // k e^{Lambda_{16w+15} - Lambda_i}
        row8f(t_eEa + w * KD + 32 * s, q, f);
      } else {
        const F3 cf = ldf3(smPb, w, s, l);           // k (e^{Lambda_64 - Lambda_i})
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = (float)cf.hi.v[e] + (float)cf.lo.v[e];
        if (scalar_g) {
#pragma unroll
          for (int e = 0; e < 8; ++e) f[e] = tokv[3 * CH + i_row];
        } else {
          row8f(t_eE64 + 32 * s, q, f);
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = lastd ? x[e] * f[e] : 0.f;
      const F3 fk = P::f3(x);
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int o = fofs(2 * s + hf, w >> 1, l) + 4 * (w & 1);
        const f32x4 ch = tr_half(fk.hi, hf, r16, q);
        const f32x4 cl = tr_half(fk.lo, hf, r16, q);
        const float xh[4] = {ch[0], ch[1], ch[2], ch[3]};
        const float xl[4] = {cl[0], cl[1], cl[2], cl[3]};
        SS::st4(smQb + o, xh);
        SS::st4(smQb + SQ + o, xl);
      }
    }
  }
  lds_barrier();
  DN_STAMP(0, 7);
  // ---- phase 6: masks; Md to the workspace, A^T into LDS --------------------
  // A strictly lower and same document; M lower and same document.
  auto mask_a = [&](f32x4& t, int rb, int cb) {   // A tile (rb, cb), lane (j, q)
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const int i = 16 * rb + 4 * q + ii, j = 16 * cb + r16;
      if (!(j < i && doc[i] == doc[j])) t[ii] = 0.f;
    }
  };
  auto store_md = [&](int blk, f32x4 m) {         // M^T tile (blk, blk), lane (i, q)
    const int i = 16 * blk + r16;
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const int j = 16 * blk + 4 * q + ii;
      if (!(j <= i && doc[i] == doc[j])) m[ii] = 0.f;
    }
    const float x[4] = {m[0], m[1], m[2], m[3]};
    const int o = fofs(blk, blk >> 1, l) + 4 * (blk & 1);
    SS::st4s(gM + o, gM + SQ + o, x);
    if (!(blk & 1)) {   // the upper half of slab blk/2 of row block blk is zero
      const float z[4] = {0.f, 0.f, 0.f, 0.f};
      SS::st4s(gM + o + 4, gM + SQ + o + 4, z);
    }
  };
#pragma unroll
  for (int cc = 0; cc < 8; ++cc)
    if (cc <= w) mask_a(At[cc], w, cc);
  store_md(w, Md);
  // A^T[j][i] = A[i][j]: tile (w, cc) lands at rows 16cc + j, columns 16w + 4q
  // (tiles above the diagonal of A, i.e. below it in A^T, are written as zeros)
#pragma unroll
  for (int cc = 0; cc < 8; ++cc) {
    const f32x4 v = (cc <= w) ? At[cc] : zero4();
    *reinterpret_cast<f32x4*>(smP + (16 * cc + r16) * TP + 16 * w + 4 * q) = v;
  }
  lds_barrier();

  DN_STAMP(0, 8);
  // ---- phase 6b: diagonal blocks whose span exceeds 2^99 (blockwise only) --
  // A_ij = sum_r bk_i k_j e^{loc_i - loc_j}, M_ij = sum_r q_i k_j e^{loc_i - loc_j}
  // summed per element; the owner reloads its rows, and the block's loc and
  // k are staged in smT for the column side.  The results replace the
  // block's diagonal tiles of A^T (LDS) and M (workspace).
  if (diag_bad) {
    float* stg = smT;                 // [2][16][128]: loc, k of the block
    float* res = smT + 4096;          // [2][16][16] A, M
#pragma unroll 1
    for (int a = 0; a < 8; ++a) {
      if (!((diag_bad >> a) & 1)) continue;
      Rows R;
      float nq2 = 0.f, nk2 = 0.f;
      if (w == a) {
        load_rows(a, R);
        norms(R, nq2, nk2);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          float gv2[8], qv[8], kv[8], bk[8];
          R.g[s].to(gv2);
          prep(R, s, nq2, nk2, valid, qv, kv, bk);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int o = r16 * KD + 32 * s + pi_k(q, e);
            stg[o] = row_scan16(r16 == 0 ? 0.f : act_g(gv2[e], valid));
            stg[2048 + o] = kv[e];
          }
        }
      }
      lds_barrier();
      if (w == a) {
        float sa[16], sm[16];
#pragma unroll
        for (int jj = 0; jj < 16; ++jj) { sa[jj] = 0.f; sm[jj] = 0.f; }
#pragma unroll 1
        for (int s = 0; s < 4; ++s) {
          float li[8], qi[8], ki[8], bi[8];
          row8f(stg + r16 * KD + 32 * s, q, li);
          prep(R, s, nq2, nk2, valid, qi, ki, bi);
#pragma unroll
          for (int jj = 0; jj < 16; ++jj) {
            float lj[8], kj[8];
            row8f(stg + jj * KD + 32 * s, q, lj);
            row8f(stg + 2048 + jj * KD + 32 * s, q, kj);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const float f = expn(fminf(li[e] - lj[e], 0.f)) * kj[e];
              sa[jj] += bi[e] * f;
              sm[jj] += qi[e] * f;
            }
          }
        }
#pragma unroll
        for (int jj = 0; jj < 16; ++jj) {
          sa[jj] += __shfl_xor(sa[jj], 16); sa[jj] += __shfl_xor(sa[jj], 32);
          sm[jj] += __shfl_xor(sm[jj], 16); sm[jj] += __shfl_xor(sm[jj], 32);
        }
        if (q == 0) {
#pragma unroll
          for (int jj = 0; jj < 16; ++jj) {
            res[r16 * 16 + jj] = sa[jj];         // A[16a + r16][16a + jj]
            res[256 + r16 * 16 + jj] = sm[jj];   // M[16a + r16][16a + jj]
          }
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wave's LDS writes
        __builtin_amdgcn_wave_barrier();
        f32x4 ta, tm;
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          ta[ii] = res[(4 * q + ii) * 16 + r16];
          tm[ii] = res[256 + r16 * 16 + 4 * q + ii];
        }
        mask_a(ta, a, a);
        store_md(a, tm);
        *reinterpret_cast<f32x4*>(smP + (16 * a + r16) * TP + 16 * a + 4 * q) = ta;
      }
      lds_barrier();
    }
  }

  // M rows were written to the workspace by other waves: a full barrier
  // (stores drained), then their loads fly during T
  __syncthreads();
  F3 MB[4];
#pragma unroll
  for (int s = 0; s < 4; ++s)
    if (s <= (am >> 1)) MB[s] = SS::fa3(gM + fofs(am, s, l), gM + SQ + fofs(am, s, l));
  DN_STAMP(0, 9);
  // ---- phase 7: T^T = (I + A^T)^-1 in place (upper unit triangular) --------
  // 16 x 16 diagonal blocks by back substitution (waves 0-1, one block per
  // 16-lane row, lane = column), then doubling Y_PQ = -Y_PP V_PQ Y_QQ for
  // block sizes 16, 32, 64 on fp32 MFMA.
  if (w < 2) {
    const int o = 16 * (4 * w + q);
    const int j = r16;
    float y[16];
#pragma unroll
    for (int i = 15; i >= 0; --i) {
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int k = i + 1; k < 16; ++k) {
        const float v = smP[(o + i) * TP + o + k];
        if (k & 1) s1 = fmaf(v, y[k], s1); else s0 = fmaf(v, y[k], s0);
      }
      y[i] = (i == j ? 1.f : 0.f) - (s0 + s1);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) smP[(o + i) * TP + o + j] = y[i];
  }
  lds_barrier();
  {
    // acc += X[r0 + 0..15][k0 .. k1) * Y[k0 .. k1)[c0 + 0..15] on fp32 MFMA
    // (k range in whole 16-blocks; lane (r, q) feeds k = k + 4q + e)
    auto tprod = [&](f32x4& acc, const float* X, int xp, int r0, const float* Y, int yp, int c0, int k0, int k1) {
      for (int k = k0; k < k1; k += 16) {
        const f32x4 av = *reinterpret_cast<const f32x4*>(X + (r0 + r16) * xp + k + 4 * q);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float bv = Y[(k + 4 * q + e) * yp + c0 + r16];
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[e], bv, acc, 0, 0, 0);
        }
      }
    };
    constexpr int WP = 68;
    float* Wsc = smT;   // W = V_PQ Y_QQ of each pair: rows pk * s ..
#pragma unroll 1
    for (int s = 16; s <= 64; s *= 2) {
      const int nt = s / 16;
      const int ntile = (CH / (2 * s)) * nt * nt;
      for (int tau = w; tau < ntile; tau += 8) {
        const int pk = tau / (nt * nt), ti = (tau / nt) % nt, tj = tau % nt;
        const int P0 = 2 * s * pk, Q0 = P0 + s;
        f32x4 acc = zero4();
        tprod(acc, smP, TP, P0 + 16 * ti, smP, TP, Q0 + 16 * tj, Q0, Q0 + 16 * (tj + 1));
        float* Wp = Wsc + pk * s * WP;
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) Wp[(16 * ti + 4 * q + ii) * WP + 16 * tj + r16] = acc[ii];
      }
      lds_barrier();
      for (int tau = w; tau < ntile; tau += 8) {
        const int pk = tau / (nt * nt), ti = (tau / nt) % nt, tj = tau % nt;
        const int P0 = 2 * s * pk, Q0 = P0 + s;
        f32x4 acc = zero4();
        const float* Wrow = Wsc + pk * s * WP - P0 * WP;   // row k of W at k - P0
        tprod(acc, smP, TP, P0 + 16 * ti, Wrow, WP, 16 * tj, P0 + 16 * ti, P0 + s);
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) smP[(P0 + 16 * ti + 4 * q + ii) * TP + Q0 + 16 * tj + r16] = -acc[ii];
      }
      lds_barrier();
    }
  }

  DN_STAMP(0, 10);
  // ---- phase 8: R^T = T^T [M^T | ke] -> R rows (split) in LDS -------------
  // TT(t, s): lane (t, q) = T[32s + pi(q, e)][16t + t] = Y[16t + t][32s + pi].
  // Wave w forms R_Q^T tiles (t, w) for every t and R_O^T tiles (t, am) for
  // t <= am; stacked in pairs of t they are the R rows of tile w (R_Q) and am
  // (R_O), which go to LDS once T^T is no longer read: R_O over smP, R_Q over
  // smQ, each [tile][slab][lane][8], high words then low words.
  bf16* Ro = reinterpret_cast<bf16*>(smP);
  bf16* Rq = smQb;
  {
    f32x4 aq[8], ao[8];
    auto TT = [&](int t, int s) -> F1 {
      float x[8];
      row8f(smP + (16 * t + r16) * TP + 32 * s, q, x);
      return P::f1(x);
    };
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      aq[t] = zero4();
      ao[t] = zero4();
#pragma unroll
      for (int s = t >> 1; s < 4; ++s) {
        const F1 tt = TT(t, s);
        P::m13(aq[t], tt, ldf3(smQb, w, s, l));
        if (t <= am && s <= (am >> 1)) P::m13(ao[t], tt, MB[s]);
      }
    }
    lds_barrier();
    auto put = [&](bf16* base, int tile, int t, const f32x4& acc) {
      const float x[4] = {acc[0], acc[1], acc[2], acc[3]};
      const int o = fofs(tile, t >> 1, l) + 4 * (t & 1);
      SS::st4s(base + o, base + SQ + o, x);
    };
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      put(Rq, w, t, aq[t]);
      if (t <= am) put(Ro, am, t, ao[t]);
    }
    if (!(am & 1)) put(Ro, am, am + 1, zero4());   // tile am+1 of R_O row block am is zero
  }
  lds_barrier();
  DN_STAMP(0, 11);

  // ---- phase 9: value products --------------------------------------------
  //   X^T(t, it) = qe^T(t, it) - sum_s be^T(t, s) R_O(it, s)   bf16
  //   Pn^T(t, rt) = -sum_s be^T(t, s) R_Q(rt, s)               bf16
  //   Oi^T(vt, it) = sum_s wv^T(vt, s) R_O(it, s)              split x split
  //   Q(rt, vt)    = sum_s R_Q(rt, s) wv(s, vt)                split x split
  // Wave w: key-channel tile w of be, value tiles [w nvw, (w+1) nvw)
  // (nvw = value tiles / 8), (w v)^T by identity transposes of v rows.
  {
    auto Rf3 = [&](const bf16* base, int tile, int s) {
      const int o = fofs(tile, s, l);
      return SS::fa3(base + o, base + SQ + o);
    };
    const int nvw = p.nct >> 3;
    {
      const bf16* Be = (const bf16*)p.BeF + u * SQ;
      F1 be[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) be[s] = SS::fa(Be + fofs(w, s, l));
      const float* Qe = p.QeC + u * SQ;
      bf16* Xh = (bf16*)p.XF + u * 2 * SQ;
      bf16* Xl = Xh + SQ;
#pragma unroll
      for (int it = 0; it < 8; ++it) {
        f32x4 acc = zero4();
#pragma unroll
        for (int s = 0; s <= (it >> 1); ++s) P::m11(acc, be[s], SS::fa(Ro + fofs(it, s, l)));
        const f32x4 qe = *reinterpret_cast<const f32x4*>(Qe + cofs(w, it, 8, l));
        const float x[4] = {qe[0] - acc[0], qe[1] - acc[1], qe[2] - acc[2], qe[3] - acc[3]};
        const int o = fofs(it, w >> 1, l) + 4 * (w & 1);
        SS::st4s(Xh + o, Xl + o, x);
      }
      bf16* Pn = (bf16*)p.PnF + u * SQ;
#pragma unroll
      for (int rt = 0; rt < 8; ++rt) {
        f32x4 acc = zero4();
#pragma unroll
        for (int s = 0; s < 4; ++s) P::m11(acc, be[s], SS::fa(Rq + fofs(rt, s, l)));
        const float x[4] = {-acc[0], -acc[1], -acc[2], -acc[3]};
        SS::st4(Pn + fofs(rt, w >> 1, l) + 4 * (w & 1), x);
      }
    }
    float* gOi = p.OiC + u * (int64_t)(CH * p.Vp);
    float* gQ = p.QCw + u * (int64_t)(KD * p.Vp);
    int vstep = 1;
#pragma unroll 1
    for (int vp = 0; vp < nvw; vp += vstep) {
      const int vt0 = w * nvw + vp;
      const bool two = vp + 1 < nvw && !(vt0 & 1);   // vt0, vt0 + 1 share one 32-column slab
      vstep = two ? 2 : 1;
      const int hv = p.gates_at_hv ? h : h * p.G + (16 * vt0) / KD;
      const int col0 = (16 * vt0) & ~31 & (KD - 1);   // 32-column slab holding vt0
      const int half0 = vt0 & 1;                       // vt0's half of that slab
      const int hw = vgate_head(p, p.w_h, hv);
      // an offset the compiler cannot prove zero keeps the R fragment reads
      // inside the loop (hoisted, all 52 would not fit in registers)
      const int zo = __builtin_amdgcn_readfirstlane(vp) & 0x40000000;
      const bf16* RoL = Ro + zo;
      const bf16* RqL = Rq + zo;
      F3 Wv[2][4];
      {
        // v and w rows of the 8 token tiles, loaded raw (converted at use)
        Raw8<TV> rv[8];
        Raw8<float> rwv[8];
        float wsc[8];
#pragma unroll
        for (int a = 0; a < 8; ++a) {
          const int t = tb + 16 * a + r16;
          const int64_t bt = (int64_t)b * p.L + min(t, t_end - 1);
          rv[a].load((const TV*)p.v + (bt * p.Hv + hv) * KD + col0, q);
          if (p.w_c == 1) {
            wsc[a] = ((const float*)p.w)[bt * p.w_h + hw];
          } else {
            rwv[a].load((const float*)p.w + (bt * p.w_h + hw) * p.w_c + col0, q);
          }
        }
#pragma unroll
        for (int a = 0; a < 8; ++a) {
          const bool ok = tb + 16 * a + r16 < t_end;
          float vv[8], ww[8];
          rv[a].to(vv);
          if (p.w_c == 1) {
#pragma unroll
            for (int e = 0; e < 8; ++e) ww[e] = wsc[a];
          } else {
            rwv[a].to(ww);
          }
          float x[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float wg = p.fuse ? sigmoid_fast(ww[e]) : ww[e];
            x[e] = ok ? wg * vv[e] : 0.f;
          }
          const F3 fx = P::f3(x);
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) {
            // Wv[0] = vt0 (half half0 of the slab), Wv[1] = vt0 + 1 (the other half)
            if (hf == 1 && !two) break;
            const int hsel = two ? hf : half0;
            const f32x4 ch = tr_half(fx.hi, hsel, r16, q);
            const f32x4 cl = tr_half(fx.lo, hsel, r16, q);
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
              Wv[hf][a >> 1].hi.v[4 * (a & 1) + ii] = (bf16)ch[ii];
              Wv[hf][a >> 1].lo.v[4 * (a & 1) + ii] = (bf16)cl[ii];
            }
          }
        }
      }
#pragma unroll
      for (int it = 0; it < 8; ++it) {
        f32x4 a0 = zero4(), a1 = zero4();
#pragma unroll
        for (int s = 0; s <= (it >> 1); ++s) {
          const F3 r = Rf3(RoL, it, s);
          P::m33(a0, Wv[0][s], r);
          if (two) P::m33(a1, Wv[1][s], r);
        }
        *reinterpret_cast<f32x4*>(gOi + cofs(vt0, it, 8, l)) = a0;
        if (two) *reinterpret_cast<f32x4*>(gOi + cofs(vt0 + 1, it, 8, l)) = a1;
      }
#pragma unroll
      for (int rt = 0; rt < 8; ++rt) {
        f32x4 a0 = zero4(), a1 = zero4();
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const F3 r = Rf3(RqL, rt, s);
          P::m33(a0, r, Wv[0][s]);
          if (two) P::m33(a1, r, Wv[1][s]);
        }
        *reinterpret_cast<f32x4*>(gQ + cofs(rt, vt0, p.nct, l)) = a0;
        if (two) *reinterpret_cast<f32x4*>(gQ + cofs(rt, vt0 + 1, p.nct, l)) = a1;
      }
    }
  }
  DN_STAMP(0, 15);
  DN_RSTAMP(0, 17);
}

// ===========================================================================
// k_scan: the sequential recurrence S' = [same doc] D S + Pn S + Q over the
// chunks of one token block.  One 4-wave workgroup per (16 state columns,
// exec head, batch); wave w holds state rows 32w .. 32w+31 in fp32 VGPRs.
// Each chunk: the entering state S_c is stored (split) for k_out, its slab is
// exchanged through LDS (high words), and Pn S (bf16) + Q + D S forms S_{c+1}.
// Operands are prefetched three chunks ahead.
// ===========================================================================
__global__ __launch_bounds__(256) void k_scan(const PF p) {
  __shared__ __align__(16) bf16 Sx[2][4 * 64 * 8];   // [buffer][slab][lane][8] high words
  __shared__ int flg[2 * 1024];
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l = tid & 63, r16 = l & 15, q = l >> 4;
  int ct, h, b;
  xcd_block(ct, h, b);
  const int hv = p.gates_at_hv ? h : h * p.G + (16 * ct) / KD;
  const int vc = (16 * ct) % KD;
  for (int i = tid; i < 2 * p.NCb; i += 256) flg[i] = p.flags[(int64_t)b * p.NCb * 2 + i];
  const int64_t sbase = ((int64_t)b * p.Hv + hv) * KD * KD + vc + r16;
  f32x4 S[2];
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int ii = 0; ii < 4; ++ii)
      S[r][ii] = p.has_init ? p.init[sbase + (int64_t)(32 * w + 16 * r + 4 * q + ii) * KD] : 0.f;
  __syncthreads();
  struct Ops {
    F1 pn[2][4];
    f32x4 qc[2], dv[2];
  };
  const int64_t ubase = ((int64_t)b * p.Hx + h) * p.NCb;
  const int64_t sfstride = (int64_t)KD * p.Vp;   // elements of one unit's S_c^T (one word)
  auto load_ops = [&](int cc, Ops& o) {
    const int64_t uu = ubase + min(cc, p.NCb - 1);
    const bf16* Pn = (const bf16*)p.PnF + uu * SQ;
    const float* Qc = p.QCw + uu * sfstride;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
#pragma unroll
      for (int s = 0; s < 4; ++s) o.pn[r][s] = SS::fa(Pn + fofs(2 * w + r, s, l));
      o.qc[r] = *reinterpret_cast<const f32x4*>(Qc + cofs(2 * w + r, ct, p.nct, l));
      o.dv[r] = *reinterpret_cast<const f32x4*>(p.dvec + uu * KD + 32 * w + 16 * r + 4 * q);
    }
  };
  auto step = [&](int cc, const Ops& o) {
    const int is_new = flg[2 * cc], same = flg[2 * cc + 1];
    if (is_new) { S[0] = zero4(); S[1] = zero4(); }
    const float x[8] = {S[0][0], S[0][1], S[0][2], S[0][3], S[1][0], S[1][1], S[1][2], S[1][3]};
    const int fo = (w * 64 + l) * 8;
    bf16* bh = &Sx[cc & 1][0];
    bf16x8 hi, lo;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      hi[e] = (bf16)x[e];
      lo[e] = (bf16)(x[e] - (float)hi[e]);
    }
    *reinterpret_cast<bf16x8*>(bh + fo) = hi;
    {
      bf16* gS = (bf16*)p.SF + (ubase + cc) * 2 * sfstride;
      const int o = fofs(ct, w, l);
      *reinterpret_cast<bf16x8*>(gS + o) = hi;
      *reinterpret_cast<bf16x8*>(gS + sfstride + o) = lo;
    }
    lds_barrier();
    F1 Sf[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) Sf[s] = SS::fa(bh + (s * 64 + l) * 8);
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      f32x4 acc = o.qc[r];
#pragma unroll
      for (int s = 0; s < 4; ++s) P::m11(acc, o.pn[r][s], Sf[s]);
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) S[r][ii] = acc[ii] + (same ? o.dv[r][ii] * S[r][ii] : 0.f);
    }
  };
  constexpr int RS = 4;
  Ops o[RS];
#pragma unroll
  for (int jj = 0; jj + 1 < RS; ++jj) load_ops(jj, o[jj]);
  const int ntrip = p.NCb / RS;
#pragma unroll 1
  for (int k = 0; k < ntrip; ++k) {
#pragma unroll
    for (int jj = 0; jj < RS; ++jj) {
      load_ops(RS * k + jj + RS - 1, o[(jj + RS - 1) % RS]);
      step(RS * k + jj, o[jj]);
    }
  }
  const int rem = p.NCb - RS * ntrip;
#pragma unroll
  for (int jj = 0; jj + 1 < RS; ++jj)
    if (jj < rem) step(RS * ntrip + jj, o[jj]);
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) p.fin[sbase + (int64_t)(32 * w + 16 * r + 4 * q + ii) * KD] = S[r][ii];
}

// ===========================================================================
// k_out: O^T(vt, it) = Oi^T(vt, it) + sum_s S_c^T(vt, s) X^T(s, it), chunk
// parallel.  One 8-wave workgroup per unit: the unit's X (split, 64 KB) is
// staged in LDS once, and wave w owns value tiles [w nvw, (w+1) nvw) with
// their S_c^T fragments in registers.  Every global load is issued before the
// first product.  Lane (i, q) holds O[token 16it + i][column 16vt + 4q + ii].
// ===========================================================================
template <class TO>
__global__ __launch_bounds__(512) void k_out(const PF p) {
  __shared__ __align__(16) bf16 Xs[2 * SQ];
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l = tid & 63, r16 = l & 15, q = l >> 4;
  const int tot = p.B * p.Hx * p.NCb;
  int id = blockIdx.x;
  if ((tot & 7) == 0) id = (id & 7) * (tot >> 3) + (id >> 3);
  const int64_t u = id;
  const int c = (int)(u % p.NCb);
  const int h = (int)((u / p.NCb) % p.Hx);
  const int b = (int)(u / ((int64_t)p.NCb * p.Hx));
  const int tb = p.t0 + c * CH;
  const int t_end = min(p.t0 + p.nt, p.L);
  const int nvw = p.nct >> 3;
  const int64_t sfstride = (int64_t)KD * p.Vp;
  {
    const uint4* src = reinterpret_cast<const uint4*>((const bf16*)p.XF + u * 2 * SQ);
    uint4* dst = reinterpret_cast<uint4*>(Xs);
    uint4 t[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) t[k] = src[k * 512 + tid];
#pragma unroll
    for (int k = 0; k < 8; ++k) dst[k * 512 + tid] = t[k];
  }
  const bf16* gS = (const bf16*)p.SF + u * 2 * sfstride;
  const float* gOi = p.OiC + u * (int64_t)(CH * p.Vp);
#pragma unroll 1
  for (int vi = 0; vi < nvw; ++vi) {
    const int vt = w * nvw + vi;
    F3 sf[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) sf[s] = SS::fa3(gS + fofs(vt, s, l), gS + sfstride + fofs(vt, s, l));
    f32x4 acc[8];
#pragma unroll
    for (int it = 0; it < 8; ++it) acc[it] = *reinterpret_cast<const f32x4*>(gOi + cofs(vt, it, 8, l));
    if (vi == 0) __syncthreads();
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int it = 0; it < 8; ++it) P::m33(acc[it], sf[s], ldf3(Xs, it, s, l));
    const int hv = p.gates_at_hv ? h : h * p.G + (16 * vt) / KD;
    const int vc = (16 * vt) % KD;
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int t = tb + 16 * it + r16;
      const bool tv = t < t_end;
      const int64_t ob = (((int64_t)b * p.L + (tv ? t : 0)) * p.Hv + hv) * KD + vc + 4 * q;
      TO* dst = tv ? (TO*)p.out + ob : (TO*)p.sink + 4 * l;
      const float x[4] = {acc[it][0], acc[it][1], acc[it][2], acc[it][3]};
      st4<TO>(dst, x);
    }
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
template <class TIn, class TV>
hipError_t launch_t(const PF& p, hipStream_t st) {
  const int units = p.B * p.Hx * p.NCb;
  prof_mark(0, st, false);
  hipLaunchKernelGGL((k_wy<TIn, TV>), dim3(units), dim3(512), 0, st, p);
  prof_mark(0, st, true);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  prof_mark(2, st, false);
  hipLaunchKernelGGL(k_scan, dim3(p.nct, p.Hx, p.B), dim3(256), 0, st, p);
  prof_mark(2, st, true);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  prof_mark(5, st, false);
  hipLaunchKernelGGL((k_out<TV>), dim3(units), dim3(512), 0, st, p);
  prof_mark(5, st, true);
  return hipGetLastError();
}

}  // namespace wy

#ifdef DN_STAMPS
extern "C" int dn_debug_stamps(unsigned long long* out) {
  return hipMemcpyFromSymbol(out, HIP_SYMBOL(wy::dn_stamp_buf), sizeof(wy::dn_stamp_buf)) == hipSuccess ? 0 : 1;
}
#endif

hipError_t launch_wy(const PF& p, hipStream_t st, int qk_dt, bool v_bf16) {
  if (qk_dt == DN_BF16) return v_bf16 ? wy::launch_t<bf16, bf16>(p, st) : wy::launch_t<bf16, float>(p, st);
  if (qk_dt == DN_F16) return v_bf16 ? wy::launch_t<f16, bf16>(p, st) : wy::launch_t<f16, float>(p, st);
  return v_bf16 ? wy::launch_t<float, bf16>(p, st) : wy::launch_t<float, float>(p, st);
}

}  // namespace dn
