// Chunked WY prefill for GDN-2 / Gated DeltaNet on gfx950 (MI355X).
//
// Reference algorithm (maelie-labs/deltanet-tpu v0.3.0, src/deltanet_tpu/):
//   prepass   gdn2.py:115-240   (Lambda, A, M, T = (I+A)^-1, W, U, qe, ke)
//   state     gdn2.py:585-652   (Vnew = U - W S, O = qe S + M Vnew,
//                                S <- [same doc] diag(e^Lend) S + ke^T Vnew)
//   flags     gdn2.py:1291-1302 (is_new_doc, all_same_doc per chunk)
//   wrapper   gdn2.py:1970-2125 (clamps, scale, L2-norm, gate broadcast,
//                                segment canonicalisation, padding)
//
// The MI355X design splits the work into three launches per token block so
// that only a 128x128-by-128x16 product sits on the sequential critical path.
// With Vnew = U - W S the reference's per-chunk update and output become
//     S_next = [same doc] diag(e^Lend) S + Pn S + Q,  Pn = -ke^T W,  Q = ke^T U
//     O      = X S + Oi,                              X = qe - M W,  Oi = M U
// so:
//   k_prepass (grid: chunk x exec-head x batch, 4 waves, one chunk each)
//       everything that is parallel over chunks: fused prologue, Lambda,
//       A and M on MFMA, T by blocked substitution on fp32 MFMA, W, U and
//       the four chunk operators Pn, Q, X, Oi.
//   k_chain   (grid: 16-column tile x exec-head x batch, 4 waves)
//       the sequential scan over chunks with the fp32 state in VGPRs;
//       stores each chunk's entry state S_c.
//   k_output  (grid: chunk x exec-head x batch, 4 waves)
//       parallel again: O = X S_c + Oi.
//
// All intermediates live in a caller-provided workspace sized for one token
// block, small enough to stay resident in the 256 MB Infinity Cache.
#include <type_traits>

#include "dn_common.h"
#include "dn_host.h"

namespace dn {

constexpr int CH = 128;   // chunk size (gdn2.py:1869)
constexpr int KD = 128;   // key / value head dim (gdn2.py:1897)
constexpr int XP = 132;   // fp32 LDS pitch (floats): conflict-free 16-lane column groups

// diag blocks whose in-block log2-decay span exceeds this use the
// overflow-free hierarchical path (e^{69} stays far inside the fp32 range)
constexpr float kDiagSafeLog2 = 100.f;

// ---------------------------------------------------------------------------
// gate activations (gdn2.py:38-47, 133-142, 1970-1974)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float act_g(float x, int fuse, int guard) {
  if (fuse) {
    x = -__expf(fminf(x, 5.f));
  } else {
    x = fminf(x, 0.f);  // _nonpositive: x <= 0 ? x : 0 (NaN -> 0)
  }
  if (guard) x = fminf(x, -1e-6f);
  return x;
}
__device__ __forceinline__ float sigmoidf_(float x) { return 1.f / (1.f + __expf(-x)); }
__device__ __forceinline__ float act_b(float x, int fuse, int guard) {
  if (fuse) return sigmoidf_(x);
  return guard ? fmaxf(x, 0.f) : x;
}
__device__ __forceinline__ float act_w(float x, int fuse) { return fuse ? sigmoidf_(x) : x; }

// head of a K-side gate (g, b) used by execution head h
__device__ __forceinline__ int kgate_head(const PF& p, int H, int h) {
  if (H == 1) return 0;
  if (p.gates_at_hv) return (H == p.Hv) ? h : h / p.G;
  return h;
}
// head of a value-side gate (w) used by value head hv
__device__ __forceinline__ int vgate_head(const PF& p, int H, int hv) {
  if (H == 1) return 0;
  return (H == p.Hv) ? hv : hv / p.G;
}

__device__ __forceinline__ int64_t seg_at(const PF& p, int b, int t) {
  const int64_t i = p.seg_batched ? (int64_t)b * p.L + t : (int64_t)t;
  return ld_i(p.seg, i, p.seg_dt);
}

template <bool BF> using MTy = typename std::conditional<BF, bf16, float>::type;

// ===========================================================================
// k_prepass: everything that is parallel over chunks (one workgroup, 4 waves,
// per (chunk, execution head, batch)).
//
// Lambda is kept block-local: X[i] = sum of g over the 16-token block of i up
// to and including i (log2 units), so a difference of two Lambdas is never
// the difference of two large cumulative sums (no fp32 cancellation after a
// strongly decayed stretch).  Cross-block factors come from the per-block
// totals: Off[a] / Suf[a] = sum of the totals before / after block a.
// ===========================================================================
template <bool BF, class TIn, class TV>
__global__ __launch_bounds__(256) void k_prepass(const PF p) {
  using P = Pol<BF>;
  using F1 = typename P::F1;
  using F3 = typename P::F3;
  using MT = MTy<BF>;
  constexpr int YP = 132;
  __shared__ float X[CH * XP];      // local Lambda (log2) -> A -> T
  __shared__ float Y[CH * YP];      // Lambda low words (1-2), Kc (2-3), w*v transposed (6)
  __shared__ float Ftab[8 * KD];    // e^{total of block b}
  __shared__ float Mid0[8 * KD];    // e^{g at the first token of block a}
  __shared__ float Off[9 * KD];     // log2: sum of totals of blocks < a (Off[8] = Lambda_end)
  __shared__ float Suf[8 * KD];     // log2: sum of totals of blocks > a
  __shared__ int doc[CH];
  __shared__ int unsafe_part[2][8];  // per 64-channel half: block needs the hierarchical path

  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63, r16 = l & 15, q = l >> 4;
  const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tb = p.t0 + c * CH;
  const int t_end = min(p.t0 + p.nt, p.L);
  const int64_t u = ((int64_t)b * p.Hx + h) * p.NCb + c;
  const int hk = p.gates_at_hv ? h / p.G : h;

  MT* g_Pn = (MT*)p.Pn + u * KD * KD;
  float* g_Q = p.Q + u * KD * p.Vp;
  float* g_X = p.X + u * CH * KD;
  float* g_Oi = p.Oi + u * CH * p.Vp;
  float* g_dv = p.dvec + u * KD;
  float* g_beT = p.beT + u * KD * CH;
  float* g_keT = p.keT + u * KD * CH;
  float* g_M = p.Mg + u * CH * CH;
  float* g_qe = p.qe + u * CH * KD;

  // ---- phase 0: in-chunk document index (segment canonicalisation) -------
  if (tid < CH) {
    int ch = 0;
    if (p.seg != nullptr && tid > 0) {
      const int t = min(tb + tid, t_end - 1), tp = min(tb + tid - 1, t_end - 1);
      ch = seg_at(p, b, t) != seg_at(p, b, tp);
    }
    doc[tid] = ch;
  }
  __syncthreads();
  for (int off = 1; off < CH; off <<= 1) {
    int v = 0;
    if (tid < CH && tid >= off) v = doc[tid - off];
    __syncthreads();
    if (tid < CH) doc[tid] += v;
    __syncthreads();
  }
  if (tid == 0 && h == 0) {
    int is_new;
    if (tb == 0) {
      if (p.has_init) {
        is_new = 0;
        if (p.init_seg != nullptr) {
          const int64_t s0 = p.seg ? seg_at(p, b, 0) : 0;
          is_new = s0 != (int64_t)p.init_seg[b];
        }
      } else {
        is_new = 1;
      }
    } else if (c == 0 && !p.has_init) {
      is_new = 1;
    } else {
      is_new = p.seg ? (seg_at(p, b, tb) != seg_at(p, b, tb - 1)) : 0;
    }
    p.flags[((int64_t)b * p.NCb + c) * 2 + 0] = is_new;
    p.flags[((int64_t)b * p.NCb + c) * 2 + 1] = (doc[CH - 1] == 0);
  }

  // ---- phase 1: block-local Lambda (double-float: X = hi, Y = lo), totals --
  {
    const int kap = tid & 127, half = tid >> 7;
    const int hg = kgate_head(p, p.g_h, h);
    // all 64 loads issued back to back: out-of-range tokens read a valid
    // address and are zeroed afterwards (no branch between the loads)
    const float* gp = (const float*)p.g;
    const int tbase = tb + 64 * half;
    float gl[64];
#pragma unroll
    for (int i = 0; i < 64; ++i) {
      const int t = min(tbase + i, t_end - 1);
      gl[i] = gp[(((int64_t)b * p.L + t) * p.g_h + hg) * p.g_c + (p.g_c == 1 ? 0 : kap)];
    }
#pragma unroll
    for (int i = 0; i < 64; ++i) gl[i] = (tbase + i < t_end) ? act_g(gl[i], p.fuse, p.guard) : 0.f;
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      float hi = 0.f, lo = 0.f;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        // error-free accumulation (TwoSum), then an exact split of hi * log2(e)
        const float gv = gl[16 * blk + j];
        const float sum = hi + gv;
        const float bb = sum - hi;
        lo += (hi - (sum - bb)) + (gv - bb);
        hi = sum;
        const float ph = hi * kLog2e;
        const float pe = fmaf(hi, kLog2e, -ph);
        const int row = 64 * half + 16 * blk + j;
        X[row * XP + kap] = ph;
        Y[row * XP + kap] = pe + lo * kLog2e;
      }
    }
  }
  __syncthreads();
  if (tid < KD) {
    float tot[8];
#pragma unroll
    for (int a = 0; a < 8; ++a) tot[a] = X[(16 * a + 15) * XP + tid] + Y[(16 * a + 15) * XP + tid];
    float acc = 0.f;
#pragma unroll
    for (int a = 0; a < 8; ++a) { Off[a * KD + tid] = acc; acc += tot[a]; }
    Off[8 * KD + tid] = acc;
    acc = 0.f;
#pragma unroll
    for (int a = 7; a >= 0; --a) { Suf[a * KD + tid] = acc; acc += tot[a]; }
#pragma unroll
    for (int a = 0; a < 8; ++a) {
      Ftab[a * KD + tid] = fast_exp2(tot[a]);
      Mid0[a * KD + tid] = fast_exp2(X[(16 * a) * XP + tid] + Y[(16 * a) * XP + tid]);
      // span of the block after its first token: Lambda(sa) - Lambda(ea) >= 0
      const int sa = 16 * a, ea = sa + 15;
      const float span = (X[sa * XP + tid] - X[ea * XP + tid]) + (Y[sa * XP + tid] - Y[ea * XP + tid]);
      const bool un = __any(span > kDiagSafeLog2);
      if (l == 0) unsafe_part[w][a] = un;
    }
    g_dv[tid] = fast_exp2(Off[8 * KD + tid]);
  }
  __syncthreads();

  // ---- phase 2: per-row quantities, diagonal A/M blocks --------------------
  F3 Rf[2][4], Qf[2][4];
  f32x4 Adiag[2];
  const int hbg = kgate_head(p, p.b_h, h);
#pragma unroll
  for (int bi = 0; bi < 2; ++bi) {
    const int a = bi == 0 ? w : 7 - w;
    const int i = 16 * a + r16;
    const int t = tb + i;
    const bool valid = t < t_end;
    float qv[32], kv[32], bet[32];
    {
      const TIn* qp = (const TIn*)p.q + (((int64_t)b * p.L + (valid ? t : 0)) * p.Hk + hk) * KD;
      const TIn* kp = (const TIn*)p.k + (((int64_t)b * p.L + (valid ? t : 0)) * p.Hk + hk) * KD;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        row8<TIn>(qp + 32 * s, q, qv + 8 * s);
        row8<TIn>(kp + 32 * s, q, kv + 8 * s);
      }
      if (!valid) {
#pragma unroll
        for (int e = 0; e < 32; ++e) { qv[e] = 0.f; kv[e] = 0.f; }
      }
      float ssq = 0.f, ssk = 0.f;
#pragma unroll
      for (int e = 0; e < 32; ++e) { ssq += qv[e] * qv[e]; ssk += kv[e] * kv[e]; }
      ssq += __shfl_xor(ssq, 16); ssq += __shfl_xor(ssq, 32);
      ssk += __shfl_xor(ssk, 16); ssk += __shfl_xor(ssk, 32);
      if (p.fuse) {
        const float rq = rsqrtf(ssq + 1e-6f), rk = rsqrtf(ssk + 1e-6f);
#pragma unroll
        for (int e = 0; e < 32; ++e) { qv[e] = (qv[e] * rq) * p.scale; kv[e] = kv[e] * rk; }
      } else if (p.l2norm) {
        const float rq = rsqrtf(ssq + 1e-6f), rk = rsqrtf(ssk + 1e-6f);
#pragma unroll
        for (int e = 0; e < 32; ++e) { qv[e] = round_as<TIn>((qv[e] * rq) * p.scale); kv[e] = round_as<TIn>(kv[e] * rk); }
      } else {
#pragma unroll
        for (int e = 0; e < 32; ++e) qv[e] = round_as<TIn>(qv[e] * p.scale);
      }
      const float* bp = (const float*)p.b + (((int64_t)b * p.L + (valid ? t : 0)) * p.b_h + hbg) * p.b_c;
      float bgv[32];
      if (p.b_c == 1) {
        const float bs = bp[0];
#pragma unroll
        for (int e = 0; e < 32; ++e) bgv[e] = bs;
      } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) row8<float>(bp + 32 * s, q, bgv + 8 * s);
      }
#pragma unroll
      for (int e = 0; e < 32; ++e) bet[e] = valid ? act_b(bgv[e], p.fuse, p.guard) * kv[e] : 0.f;
    }
    const bool first = doc[i] == 0;
    const bool last = doc[i] == doc[CH - 1];
    const bool blk_unsafe = unsafe_part[0][a] | unsafe_part[1][a];
    float dq = 0.f;
    f32x4 accA = zero4(), accM = zero4();
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      float lam[8], lsa[8], ta[8], laml[8], lsal[8], tal[8], off[8], suf[8];
      row8<float>(&X[i * XP + 32 * s], q, lam);
      row8<float>(&X[(16 * a) * XP + 32 * s], q, lsa);
      row8<float>(&X[(16 * a + 15) * XP + 32 * s], q, ta);
      row8<float>(&Y[i * XP + 32 * s], q, laml);
      row8<float>(&Y[(16 * a) * XP + 32 * s], q, lsal);
      row8<float>(&Y[(16 * a + 15) * XP + 32 * s], q, tal);
      row8<float>(&Off[a * KD + 32 * s], q, off);
      row8<float>(&Suf[a * KD + 32 * s], q, suf);
      float rA[8], rM[8], bd[8], kc[8], qe[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int kap = 32 * s + pi_k(q, e);
        const float qh = qv[8 * s + e], kh = kv[8 * s + e], be = bet[8 * s + e];
        const float d_i_sa = (lam[e] - lsa[e]) + (laml[e] - lsal[e]);   // <= 0
        const float d_ea_i = (ta[e] - lam[e]) + (tal[e] - laml[e]);     // <= 0
        const float er = fast_exp2(d_i_sa);
        rA[e] = be * er;
        rM[e] = qh * er;
        kc[e] = kh * fast_exp2(d_ea_i);
        const float eL = fast_exp2(off[e] + (lam[e] + laml[e]));
        g_beT[(int64_t)kap * CH + i] = first ? be * eL : 0.f;
        g_keT[(int64_t)kap * CH + i] = last ? kh * fast_exp2(suf[e] + d_ea_i) : 0.f;
        bd[e] = kh * fast_exp2(-d_i_sa);
        dq += qh * kh;
        qe[e] = first ? qh * eL : 0.f;
      }
      st4<float>(g_qe + (int64_t)i * KD + 32 * s + 4 * q, qe);
      st4<float>(g_qe + (int64_t)i * KD + 32 * s + 16 + 4 * q, qe + 4);
      Rf[bi][s] = P::f3(rA);
      Qf[bi][s] = P::f3(rM);
      if (!blk_unsafe) {
        // A_aa, M_aa = (R, Qr) (k e^{Lambda_sa - Lambda})^T: every factor stays
        // within 2^{+-100} of 1, so the factorisation cannot overflow.  Kc
        // replaces this slab of the row's Lambda low words once all lanes of
        // the wave have read it (the other slabs' columns are untouched).
        const F3 fb = P::f3(bd);
        P::m33(accA, Rf[bi][s], fb);
        P::m33(accM, Qf[bi][s], fb);
        st4<float>(&Y[i * YP + 32 * s + 4 * q], kc);
        st4<float>(&Y[i * YP + 32 * s + 16 + 4 * q], kc + 4);
      }
    }
    dq += __shfl_xor(dq, 16);
    dq += __shfl_xor(dq, 32);

    if (blk_unsafe) {
      // Overflow-free hierarchical factorisation: the pair (i, j) is split at
      // the highest bit where the in-block indices differ; rows above and
      // columns below the split point are scaled toward it, so every
      // exponent is <= 0.
#pragma unroll
      for (int hl = 3; hl >= 0; --hl) {
        const int hh = 1 << hl;
        const int sp = (r16 / (2 * hh)) * 2 * hh + hh;
        const bool upper = r16 >= sp;
        const int srow = 16 * a + sp;
        f32x4 tA = zero4(), tM = zero4();
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          float lam[8], lsp[8], laml[8], lspl[8], xa[8], xm[8], xb[8];
          row8<float>(&X[i * XP + 32 * s], q, lam);
          row8<float>(&X[srow * XP + 32 * s], q, lsp);
          row8<float>(&Y[i * XP + 32 * s], q, laml);
          row8<float>(&Y[srow * XP + 32 * s], q, lspl);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float d = (lam[e] - lsp[e]) + (laml[e] - lspl[e]);
            const float x = fast_exp2(upper ? d : -d);
            xa[e] = upper ? bet[8 * s + e] * x : 0.f;
            xm[e] = upper ? qv[8 * s + e] * x : 0.f;
            xb[e] = upper ? 0.f : kv[8 * s + e] * x;
          }
          const F3 fb = P::f3(xb);
          P::m33(tA, P::f3(xa), fb);
          P::m33(tM, P::f3(xm), fb);
        }
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          const int il = 4 * q + ii;
          const int d = il ^ r16;
          if (il > r16 && (31 - __builtin_clz(d)) == hl) { accA[ii] = tA[ii]; accM[ii] = tM[ii]; }
        }
      }
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
        if (4 * q + ii == r16) accM[ii] = dq;
      // Kc of this block's rows, written after every lane has read the rows'
      // Lambda low words
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        float lam[8], ta[8], laml[8], tal[8], kc[8];
        row8<float>(&X[i * XP + 32 * s], q, lam);
        row8<float>(&X[(16 * a + 15) * XP + 32 * s], q, ta);
        row8<float>(&Y[i * XP + 32 * s], q, laml);
        row8<float>(&Y[(16 * a + 15) * XP + 32 * s], q, tal);
#pragma unroll
        for (int e = 0; e < 8; ++e) kc[e] = kv[8 * s + e] * fast_exp2((ta[e] - lam[e]) + (tal[e] - laml[e]));
        st4<float>(&Y[i * YP + 32 * s + 4 * q], kc);
        st4<float>(&Y[i * YP + 32 * s + 16 + 4 * q], kc + 4);
      }
    }
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const int il = 4 * q + ii, ia = 16 * a + il, ja = 16 * a + r16;
      const bool same = doc[ia] == doc[ja];
      Adiag[bi][ii] = (il > r16 && same) ? accA[ii] : 0.f;
      g_M[(int64_t)ia * CH + ja] = (il >= r16 && same) ? accM[ii] : 0.f;
      if ((a & 1) == 0) g_M[(int64_t)ia * CH + ja + 16] = 0.f;
    }
  }
  __syncthreads();

  // ---- phase 3: off-diagonal A/M blocks (X becomes A) -----------------------
#pragma unroll
  for (int bi = 0; bi < 2; ++bi) {
    const int a = bi == 0 ? w : 7 - w;
    float mloc[32];
#pragma unroll
    for (int s = 0; s < 4; ++s) row8<float>(&Mid0[a * KD + 32 * s], q, mloc + 8 * s);
    for (int bb = a - 1; bb >= 0; --bb) {
      f32x4 accA = zero4(), accM = zero4();
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        float x[8];
        row8<float>(&Y[(16 * bb + r16) * YP + 32 * s], q, x);
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] *= mloc[8 * s + e];
        const F3 fb = P::f3(x);
        P::m33(accA, Rf[bi][s], fb);
        P::m33(accM, Qf[bi][s], fb);
      }
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int ia = 16 * a + 4 * q + ii, jb = 16 * bb + r16;
        const bool same = doc[ia] == doc[jb];
        X[ia * XP + jb] = same ? accA[ii] : 0.f;
        g_M[(int64_t)ia * CH + jb] = same ? accM[ii] : 0.f;
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        float f[8];
        row8<float>(&Ftab[bb * KD + 32 * s], q, f);
#pragma unroll
        for (int e = 0; e < 8; ++e) mloc[8 * s + e] *= f[e];
      }
    }
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const int ia = 16 * a + 4 * q + ii;
      X[ia * XP + 16 * a + r16] = Adiag[bi][ii];
      if ((a & 1) == 0) X[ia * XP + 16 * a + 16 + r16] = 0.f;
    }
  }
  __syncthreads();

  // ---- phase 4: T = (I + A)^-1 (blocked forward substitution, fp32) -------
  if (w < 2) {
    const int a = 4 * w + q;
    float tc[16];
#pragma unroll
    for (int m = 0; m < 16; ++m) tc[m] = (m == r16) ? 1.f : 0.f;
#pragma unroll
    for (int ii = 1; ii < 16; ++ii) {
      float acc = 0.f;
#pragma unroll
      for (int m = 0; m < ii; ++m) acc += X[(16 * a + ii) * XP + 16 * a + m] * tc[m];
      if (ii > r16) tc[ii] = -acc;
    }
#pragma unroll
    for (int ii = 0; ii < 16; ++ii) X[(16 * a + ii) * XP + 16 * a + r16] = tc[ii];
  }
  __syncthreads();
  for (int a = 1; a < 8; ++a) {
    f32x4 res[2];
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      const int bt = w + 4 * k2;
      res[k2] = zero4();
      if (bt < a) {
        f32x4 acc = zero4();
        for (int cc = bt; cc < a; ++cc) {
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) {
            const float av = X[(16 * a + r16) * XP + 16 * cc + 4 * kk + q];
            const float bv = X[(16 * cc + 4 * kk + q) * XP + 16 * bt + r16];
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc, 0, 0, 0);
          }
        }
        f32x4 r = zero4();
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const float av = X[(16 * a + r16) * XP + 16 * a + 4 * q + kk];
          r = __builtin_amdgcn_mfma_f32_16x16x4f32(av, acc[kk], r, 0, 0, 0);
        }
        res[k2] = -r;
      }
    }
    __syncthreads();
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      const int bt = w + 4 * k2;
      if (bt < a) {
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) X[(16 * a + 4 * q + ii) * XP + 16 * bt + r16] = res[k2][ii];
      }
    }
    __syncthreads();
  }

  // ---- phase 5: W = T be ; Pn = -ke^T W ; X = qe - M W  (key tiles w, w+4) ---
  {
    f32x4 Wc[2][8];
    F1 Bbe[2][4];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int n = 16 * (w + 4 * nt) + r16;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        float x[8];
        row8<float>(g_beT + (int64_t)n * CH + 32 * s, q, x);
        Bbe[nt][s] = P::f1(x);
      }
#pragma unroll
      for (int rt = 0; rt < 8; ++rt) Wc[nt][rt] = zero4();
    }
#pragma unroll
    for (int rt = 0; rt < 8; ++rt) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        if (s <= rt / 2) {
          float x[8];
          row8<float>(&X[(16 * rt + r16) * XP + 32 * s], q, x);
          const F1 fa = P::f1(x);
          P::m11(Wc[0][rt], fa, Bbe[0][s]);
          P::m11(Wc[1][rt], fa, Bbe[1][s]);
        }
      }
    }
    F3 W3[2][4];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const float x[8] = {Wc[nt][2 * s][0], Wc[nt][2 * s][1], Wc[nt][2 * s][2], Wc[nt][2 * s][3],
                            Wc[nt][2 * s + 1][0], Wc[nt][2 * s + 1][1], Wc[nt][2 * s + 1][2], Wc[nt][2 * s + 1][3]};
        W3[nt][s] = P::f3(x);
      }
    // rows of ke^T / M are read from the (L2-resident) scratch one step ahead
    float kx[2][32];
    auto ld_rows = [&](const float* base, int row, int nslab, float* x) {
#pragma unroll
      for (int s = 0; s < 4; ++s)
        if (s < nslab) row8<float>(base + (int64_t)row * CH + 32 * s, q, x + 8 * s);
    };
    ld_rows(g_keT, r16, 4, kx[0]);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      if (m < 7) ld_rows(g_keT, 16 * (m + 1) + r16, 4, kx[(m + 1) & 1]);
      f32x4 P0 = zero4(), P1 = zero4();
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const F1 fa = P::f1(kx[m & 1] + 8 * s);
        P::m11(P0, fa, P::hi(W3[0][s]));
        P::m11(P1, fa, P::hi(W3[1][s]));
      }
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int64_t row = (int64_t)(16 * m + 4 * q + ii) * KD;
        g_Pn[row + 16 * w + r16] = from_f<MT>(-P0[ii]);
        g_Pn[row + 16 * (w + 4) + r16] = from_f<MT>(-P1[ii]);
      }
    }
    float qx[2][8];
    auto ld_qe = [&](int rt, float* x) {
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int64_t row = (int64_t)(16 * rt + 4 * q + ii) * KD;
        x[ii] = g_qe[row + 16 * w + r16];
        x[4 + ii] = g_qe[row + 16 * (w + 4) + r16];
      }
    };
    ld_rows(g_M, r16, 1, kx[0]);
    ld_qe(0, qx[0]);
#pragma unroll
    for (int rt = 0; rt < 8; ++rt) {
      if (rt < 7) {
        ld_rows(g_M, 16 * (rt + 1) + r16, (rt + 1) / 2 + 1, kx[(rt + 1) & 1]);
        ld_qe(rt + 1, qx[(rt + 1) & 1]);
      }
      f32x4 X0, X1;
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) { X0[ii] = qx[rt & 1][ii]; X1[ii] = qx[rt & 1][4 + ii]; }
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        if (s <= rt / 2) {
          float x[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] = -kx[rt & 1][8 * s + e];
          const F3 fa = P::f3(x);
          P::m33(X0, fa, W3[0][s]);
          P::m33(X1, fa, W3[1][s]);
        }
      }
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int64_t row = (int64_t)(16 * rt + 4 * q + ii) * KD;
        g_X[row + 16 * w + r16] = X0[ii];
        g_X[row + 16 * (w + 4) + r16] = X1[ii];
      }
    }
  }

  // ---- phase 6: U = T (w*v) ; Q = ke^T U ; Oi = M U  (128 value columns per pass)
  for (int n0 = 0; n0 < p.Vp; n0 += 128) {
    __syncthreads();
    {
      // w*v for 128 tokens x 128 columns, transposed into Y[col][token]
      const int tok = tid >> 1, half = tid & 1;
      const int t = tb + tok;
      const int hv = p.gates_at_hv ? h : h * p.G + n0 / KD;
      const int hw = vgate_head(p, p.w_h, hv);
      const bool valid = t < t_end;
      const int64_t bt = (int64_t)b * p.L + (valid ? t : tb);
      const TV* vp = (const TV*)p.v + (bt * p.Hv + hv) * KD + 64 * half;
      const float* wp = (const float*)p.w + (bt * p.w_h + hw) * p.w_c;
      float vv[64], ww[64];
#pragma unroll
      for (int j = 0; j < 16; ++j) ld4<TV>(vp + 4 * j, vv + 4 * j);
      if (p.w_c == 1) {
        const float ws = wp[0];
#pragma unroll
        for (int j = 0; j < 64; ++j) ww[j] = ws;
      } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) ld4<float>(wp + 64 * half + 4 * j, ww + 4 * j);
      }
#pragma unroll
      for (int j = 0; j < 64; ++j) Y[(64 * half + j) * YP + tok] = valid ? act_w(ww[j], p.fuse) * vv[j] : 0.f;
    }
    __syncthreads();
    f32x4 Uc[2][8];
    F3 Bwv[2][4];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int col = 16 * (w + 4 * nt) + r16;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        float x[8];
        row8<float>(&Y[col * YP + 32 * s], q, x);
        Bwv[nt][s] = P::f3(x);
      }
#pragma unroll
      for (int rt = 0; rt < 8; ++rt) Uc[nt][rt] = zero4();
    }
#pragma unroll
    for (int rt = 0; rt < 8; ++rt) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        if (s <= rt / 2) {
          float x[8];
          row8<float>(&X[(16 * rt + r16) * XP + 32 * s], q, x);
          const F1 fa = P::f1(x);
          P::m13(Uc[0][rt], fa, Bwv[0][s]);
          P::m13(Uc[1][rt], fa, Bwv[1][s]);
        }
      }
    }
    F3 U3[2][4];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const float x[8] = {Uc[nt][2 * s][0], Uc[nt][2 * s][1], Uc[nt][2 * s][2], Uc[nt][2 * s][3],
                            Uc[nt][2 * s + 1][0], Uc[nt][2 * s + 1][1], Uc[nt][2 * s + 1][2], Uc[nt][2 * s + 1][3]};
        U3[nt][s] = P::f3(x);
      }
    const int c0 = n0 + 16 * w + r16, c1 = n0 + 16 * (w + 4) + r16;
    float kx[2][32];
    auto ld_rows = [&](const float* base, int row, int nslab, float* x) {
#pragma unroll
      for (int s = 0; s < 4; ++s)
        if (s < nslab) row8<float>(base + (int64_t)row * CH + 32 * s, q, x + 8 * s);
    };
    ld_rows(g_keT, r16, 4, kx[0]);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      if (m < 7) ld_rows(g_keT, 16 * (m + 1) + r16, 4, kx[(m + 1) & 1]);
      else ld_rows(g_M, r16, 1, kx[0]);
      f32x4 Q0 = zero4(), Q1 = zero4();
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const F3 fa = P::f3(kx[m & 1] + 8 * s);
        P::m33(Q0, fa, U3[0][s]);
        P::m33(Q1, fa, U3[1][s]);
      }
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int64_t row = (int64_t)(16 * m + 4 * q + ii) * p.Vp;
        g_Q[row + c0] = Q0[ii];
        g_Q[row + c1] = Q1[ii];
      }
    }
    // two row tiles per iteration (static prefetch buffers) without unrolling
    // the whole loop, so the scheduler cannot hoist every row's loads at once
    auto oi_tile = [&](int rt, const float* xcur) {
      f32x4 O0 = zero4(), O1 = zero4();
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        if (s <= rt / 2) {
          const F3 fa = P::f3(xcur + 8 * s);
          P::m33(O0, fa, U3[0][s]);
          P::m33(O1, fa, U3[1][s]);
        }
      }
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int64_t row = (int64_t)(16 * rt + 4 * q + ii) * p.Vp;
        g_Oi[row + c0] = O0[ii];
        g_Oi[row + c1] = O1[ii];
      }
    };
#pragma unroll 1
    for (int rt = 0; rt < 8; rt += 2) {
      ld_rows(g_M, 16 * (rt + 1) + r16, (rt + 1) / 2 + 1, kx[1]);
      oi_tile(rt, kx[0]);
      if (rt + 2 < 8) ld_rows(g_M, 16 * (rt + 2) + r16, (rt + 2) / 2 + 1, kx[0]);
      oi_tile(rt + 1, kx[1]);
    }
  }
}

// ===========================================================================
// k_chain: S_{c+1} = [same doc] D_c S_c + Pn_c S_c + Q_c.
// One workgroup per (16-column tile, exec head, batch); wave w owns state rows
// 32w..32w+31 (fp32, in VGPRs); the full S_c is exchanged through LDS each
// chunk so that only 8 MFMAs per wave sit on the sequential path.
// ===========================================================================
template <bool BF>
__global__ __launch_bounds__(256) void k_chain(const PF p) {
  using P = Pol<BF>;
  using F1 = typename P::F1;
  using MT = MTy<BF>;
  __shared__ float Sx[2][16 * XP];   // S^T of the current chunk, double-buffered
  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63, r16 = l & 15, q = l >> 4;
  const int ct = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int n = 16 * ct + r16;
  const int hv = p.gates_at_hv ? h : h * p.G + n / KD;
  const int vcol = n % KD;
  const int64_t sbase = ((int64_t)b * p.Hv + hv) * KD * KD + vcol;

  f32x4 S[2];
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int ii = 0; ii < 4; ++ii)
      S[r][ii] = p.has_init ? p.init[sbase + (int64_t)(32 * w + 16 * r + 4 * q + ii) * KD] : 0.f;

  // operands of chunk c, prefetched one chunk ahead
  auto load_ops = [&](int c, F1 (&pf)[2][4], f32x4 (&qc)[2], float (&dv)[8], int& is_new, int& same) {
    const int64_t u = ((int64_t)b * p.Hx + h) * p.NCb + c;
    const MT* Pn = (const MT*)p.Pn + u * KD * KD;
    const float* Qc = p.Q + u * KD * p.Vp;
    const float* dvp = p.dvec + u * KD;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        float x[8];
        row8<MT>(Pn + (int64_t)(32 * w + 16 * r + r16) * KD + 32 * s, q, x);
        pf[r][s] = P::f1(x);
      }
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) qc[r][ii] = Qc[(int64_t)(32 * w + 16 * r + 4 * q + ii) * p.Vp + n];
      ld4<float>(dvp + 32 * w + 16 * r + 4 * q, dv + 4 * r);
    }
    is_new = p.flags[((int64_t)b * p.NCb + c) * 2 + 0];
    same = p.flags[((int64_t)b * p.NCb + c) * 2 + 1];
  };

  F1 pf[2][4];
  f32x4 qc[2];
  float dv[8];
  int is_new = 0, same = 0;
  load_ops(0, pf, qc, dv, is_new, same);
  for (int c = 0; c < p.NCb; ++c) {
    const int64_t u = ((int64_t)b * p.Hx + h) * p.NCb + c;
    if (is_new) { S[0] = zero4(); S[1] = zero4(); }
    float* sx = Sx[c & 1];
    float* st = p.St + u * (int64_t)p.Vp * KD + (int64_t)n * KD;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const float x[4] = {S[r][0], S[r][1], S[r][2], S[r][3]};
      st4<float>(&sx[r16 * XP + 32 * w + 16 * r + 4 * q], x);
      st4<float>(st + 32 * w + 16 * r + 4 * q, x);
    }
    // next chunk's operands while this chunk's exchange completes
    F1 pf_n[2][4];
    f32x4 qc_n[2];
    float dv_n[8];
    int is_new_n = 0, same_n = 0;
    if (c + 1 < p.NCb) load_ops(c + 1, pf_n, qc_n, dv_n, is_new_n, same_n);
    lds_barrier();
    F1 Sf[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      float x[8];
      row8<float>(&sx[r16 * XP + 32 * s], q, x);
      Sf[s] = P::f1(x);
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      f32x4 acc = qc[r];
#pragma unroll
      for (int s = 0; s < 4; ++s) P::m11(acc, pf[r][s], Sf[s]);
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) S[r][ii] = acc[ii] + (same ? dv[4 * r + ii] * S[r][ii] : 0.f);
    }
    if (c + 1 < p.NCb) {
#pragma unroll
      for (int r = 0; r < 2; ++r) {
#pragma unroll
        for (int s = 0; s < 4; ++s) pf[r][s] = pf_n[r][s];
        qc[r] = qc_n[r];
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) dv[e] = dv_n[e];
      is_new = is_new_n;
      same = same_n;
    }
  }
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) p.fin[sbase + (int64_t)(32 * w + 16 * r + 4 * q + ii) * KD] = S[r][ii];
}

// ===========================================================================
// k_output: O_c = X_c S_c + Oi_c  (one workgroup per chunk and 256 value
// columns; each wave owns 64 columns).  X S is a split-bf16 product in
// bf16 mode.
// ===========================================================================
template <bool BF>
__global__ __launch_bounds__(256) void k_output(const PF p) {
  using P = Pol<BF>;
  using F3 = typename P::F3;
  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63, r16 = l & 15, q = l >> 4;
  const int c = blockIdx.x, h = blockIdx.y;
  const int b = blockIdx.z / p.ncg, cg = blockIdx.z % p.ncg;
  const int col0 = 256 * cg + 64 * w;
  if (col0 >= p.Vp) return;
  const int tb = p.t0 + c * CH;
  const int t_end = min(p.t0 + p.nt, p.L);
  const int64_t u = ((int64_t)b * p.Hx + h) * p.NCb + c;
  const float* Xc = p.X + u * CH * KD;
  const float* Oi = p.Oi + u * CH * p.Vp;
  const float* St = p.St + u * (int64_t)p.Vp * KD;

  F3 Sf[4][4];
  int ncol[4];
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    ncol[ct] = col0 + 16 * ct + r16;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      float x[8];
      row8<float>(St + (int64_t)ncol[ct] * KD + 32 * s, q, x);
      Sf[ct][s] = P::f3(x);
    }
  }
  const int hv = p.gates_at_hv ? h : h * p.G + col0 / KD;
  const int vcol0 = col0 % KD;
  // X rows and Oi tiles of row tile rt+1 are loaded while rt computes
  float xr[2][32], oi[2][16];
  auto ld = [&](int rt, float* x, float* o) {
#pragma unroll
    for (int s = 0; s < 4; ++s) row8<float>(Xc + (int64_t)(16 * rt + r16) * KD + 32 * s, q, x + 8 * s);
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) o[4 * ct + ii] = Oi[(int64_t)(16 * rt + 4 * q + ii) * p.Vp + ncol[ct]];
  };
  ld(0, xr[0], oi[0]);
#pragma unroll
  for (int rt = 0; rt < 8; ++rt) {
    if (rt < 7) ld(rt + 1, xr[(rt + 1) & 1], oi[(rt + 1) & 1]);
    f32x4 O[4];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) O[ct][ii] = oi[rt & 1][4 * ct + ii];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const F3 fa = P::f3(xr[rt & 1] + 8 * s);
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) P::m33(O[ct], fa, Sf[ct][s]);
    }
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const int t = tb + 16 * rt + 4 * q + ii;
      if (t < t_end) {
        const int64_t ob = (((int64_t)b * p.L + t) * p.Hv + hv) * KD + vcol0 + r16;
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
          const int64_t oi_ = ob + 16 * ct;
          if (p.v_dt == DT_BF16) ((bf16*)p.out)[oi_] = (bf16)O[ct][ii];
          else ((float*)p.out)[oi_] = O[ct][ii];
        }
      }
    }
  }
}

// ===========================================================================
// host side
// ===========================================================================
namespace {

struct WsLayout {
  size_t flags, dvec, Pn, Q, X, Oi, St, beT, keT, Mg, qe, carry, total;
};

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

WsLayout ws_layout(const dn_prefill_args* a, int Hx, int Vp, int NCb, bool bf) {
  WsLayout L{};
  const size_t es = bf ? 2 : 4;
  const size_t units = (size_t)a->B * Hx * NCb;
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off += align256(bytes); return o; };
  L.flags = take((size_t)a->B * NCb * 2 * 4);
  L.dvec = take(units * KD * 4);
  L.Pn = take(units * KD * KD * es);
  L.Q = take(units * KD * Vp * 4);
  L.X = take(units * CH * KD * 4);
  L.Oi = take(units * CH * Vp * 4);
  L.St = take(units * (size_t)Vp * KD * 4);
  L.beT = take(units * KD * CH * 4);
  L.keT = take(units * KD * CH * 4);
  L.Mg = take(units * CH * CH * 4);
  L.qe = take(units * CH * KD * 4);
  L.carry = take((size_t)a->B * a->Hv * KD * KD * 4);
  L.total = off;
  return L;
}

constexpr size_t kAutoBudget = size_t(160) << 20;

int block_chunks(const dn_prefill_args* a, int Hx, int Vp) {
  const int nct = (a->nt + CH - 1) / CH;
  if (a->block_tokens > 0) return std::max(1, std::min(nct, a->block_tokens / CH));
  const bool bf = a->precision == 0;
  int ncb = nct;
  while (ncb > 1 && ws_layout(a, Hx, Vp, ncb, bf).total > kAutoBudget) ncb = (ncb + 1) / 2;
  return std::max(1, ncb);
}

int check_args(const dn_prefill_args* a) {
  if (a == nullptr) return set_error(DN_E_INVALID, "null args");
  if (a->abi_version != DN_ABI_VERSION) return set_error(DN_E_ABI, "dn_prefill_args built for another ABI version");
  if (a->K != KD || a->V != KD) return set_error(DN_E_INVALID, "K and V must both be 128");
  if (a->B <= 0 || a->L <= 0 || a->Hk <= 0 || a->Hv <= 0) return set_error(DN_E_INVALID, "non-positive dimension");
  if (a->Hv % a->Hk != 0) return set_error(DN_E_INVALID, "Hv must be a multiple of Hk");
  if (a->t0 < 0 || a->t0 % CH != 0 || a->nt <= 0 || a->t0 + a->nt > a->L)
    return set_error(DN_E_INVALID, "token range must satisfy 0 <= t0 < t0+nt <= L with t0 % 128 == 0");
  if (!a->q || !a->k || !a->v || !a->g || !a->b || !a->w || !a->out)
    return set_error(DN_E_INVALID, "missing tensor pointer");
  if (a->qk_dtype < DN_F32 || a->qk_dtype > DN_F16)
    return set_error(DN_E_INVALID, "q/k dtype must be f32, bf16 or f16");
  if (a->v_dtype != DN_F32 && a->v_dtype != DN_BF16)
    return set_error(DN_E_INVALID, "v dtype must be f32 or bf16");
  const int G = a->Hv / a->Hk;
  auto gate_ok = [&](int H, int Cc, int dt, int full) {
    return (H == 1 || H == a->Hk || H == a->Hv) && (Cc == 1 || Cc == full) && dt == DN_F32;
  };
  if (!gate_ok(a->g_heads, a->g_chans, a->g_dtype, a->K) || !gate_ok(a->b_heads, a->b_chans, a->b_dtype, a->K) ||
      !gate_ok(a->w_heads, a->w_chans, a->w_dtype, a->V))
    return set_error(DN_E_INVALID, "gates must be float32 with 1, Hk or Hv heads and 1 or 128 channels");
  if (!a->gates_at_hv && G > 1 && (a->g_heads == a->Hv || a->b_heads == a->Hv))
    return set_error(DN_E_INVALID, "g or b has Hv heads: gates_at_hv must be set");
  if (a->seg && a->seg_dtype != DN_I32 && a->seg_dtype != DN_I64) return set_error(DN_E_INVALID, "segment ids must be int32 or int64");
  if (a->precision != 0 && a->precision != 1) return set_error(DN_E_INVALID, "precision must be 0 (bf16) or 1 (fp32)");
  if (a->block_tokens < 0 || a->block_tokens % CH != 0) return set_error(DN_E_INVALID, "block_tokens must be a multiple of 128");
  return DN_OK;
}

template <bool BF, class TIn, class TV>
hipError_t launch_all(const PF& p, hipStream_t st) {
  prof_mark(0, st, false);
  hipLaunchKernelGGL((k_prepass<BF, TIn, TV>), dim3(p.NCb, p.Hx, p.B), dim3(256), 0, st, p);
  prof_mark(0, st, true);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  prof_mark(1, st, false);
  hipLaunchKernelGGL((k_chain<BF>), dim3(p.Vp / 16, p.Hx, p.B), dim3(256), 0, st, p);
  prof_mark(1, st, true);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  prof_mark(2, st, false);
  hipLaunchKernelGGL((k_output<BF>), dim3(p.NCb, p.Hx, p.B * p.ncg), dim3(256), 0, st, p);
  prof_mark(2, st, true);
  return hipGetLastError();
}

template <bool BF, class TIn>
hipError_t dispatch_v(const PF& p, hipStream_t st, bool v_bf16) {
  return v_bf16 ? launch_all<BF, TIn, bf16>(p, st) : launch_all<BF, TIn, float>(p, st);
}

template <bool BF>
hipError_t dispatch_qk(const PF& p, hipStream_t st, int qk_dt, bool v_bf16) {
  if (qk_dt == DN_BF16) return dispatch_v<BF, bf16>(p, st, v_bf16);
  if (qk_dt == DN_F16) return dispatch_v<BF, f16>(p, st, v_bf16);
  return dispatch_v<BF, float>(p, st, v_bf16);
}

hipError_t dispatch(const PF& p, hipStream_t st, bool bf, int qk_dt, bool v_bf16) {
  return bf ? dispatch_qk<true>(p, st, qk_dt, v_bf16) : dispatch_qk<false>(p, st, qk_dt, v_bf16);
}

}  // namespace

}  // namespace dn

using namespace dn;

extern "C" size_t dn_prefill_workspace_size(const dn_prefill_args* a) {
  if (check_args(a) != DN_OK) return 0;
  const int G = a->Hv / a->Hk;
  const int Hx = a->gates_at_hv ? a->Hv : a->Hk;
  const int Vp = a->gates_at_hv ? KD : G * KD;
  return ws_layout(a, Hx, Vp, block_chunks(a, Hx, Vp), a->precision == 0).total;
}

extern "C" int dn_prefill_fwd(const dn_prefill_args* a, void* workspace, size_t workspace_bytes, void* stream) {
  const int rc = check_args(a);
  if (rc != DN_OK) return rc;
  const int G = a->Hv / a->Hk;
  const int Hx = a->gates_at_hv ? a->Hv : a->Hk;
  const int Vp = a->gates_at_hv ? KD : G * KD;
  if (Vp % 64 != 0 || Vp > 1024) return set_error(DN_E_INVALID, "value width per execution head must be 64..1024");
  const bool bf = a->precision == 0;
  const int ncb = block_chunks(a, Hx, Vp);
  const WsLayout Lw = ws_layout(a, Hx, Vp, ncb, bf);
  if (workspace == nullptr || workspace_bytes < Lw.total) return set_error(DN_E_WORKSPACE, "workspace too small");
  char* ws = (char*)workspace;

  PF p{};
  p.B = a->B; p.L = a->L; p.Hk = a->Hk; p.Hv = a->Hv; p.G = G; p.Hx = Hx; p.Vp = Vp;
  p.gates_at_hv = a->gates_at_hv;
  p.q = a->q; p.k = a->k; p.v = a->v; p.v_dt = a->v_dtype;
  p.g = a->g; p.g_dt = a->g_dtype; p.g_h = a->g_heads; p.g_c = a->g_chans;
  p.b = a->b; p.b_dt = a->b_dtype; p.b_h = a->b_heads; p.b_c = a->b_chans;
  p.w = a->w; p.w_dt = a->w_dtype; p.w_h = a->w_heads; p.w_c = a->w_chans;
  p.seg = a->seg; p.seg_dt = a->seg_dtype; p.seg_batched = a->seg_batched;
  p.init_seg = a->init_seg;
  p.out = a->out;
  p.scale = a->scale; p.l2norm = a->qk_l2norm; p.fuse = a->fuse_prologue; p.guard = a->stability_guard;
  p.ncg = (Vp + 255) / 256;
  p.flags = (int32_t*)(ws + Lw.flags);
  p.dvec = (float*)(ws + Lw.dvec);
  p.Pn = ws + Lw.Pn;
  p.Q = (float*)(ws + Lw.Q);
  p.X = (float*)(ws + Lw.X);
  p.Oi = (float*)(ws + Lw.Oi);
  p.St = (float*)(ws + Lw.St);
  p.beT = (float*)(ws + Lw.beT);
  p.keT = (float*)(ws + Lw.keT);
  p.Mg = (float*)(ws + Lw.Mg);
  p.qe = (float*)(ws + Lw.qe);
  float* carry = a->final_state ? a->final_state : (float*)(ws + Lw.carry);

  hipStream_t st = (hipStream_t)stream;
  const int t_stop = a->t0 + a->nt;
  for (int tb = a->t0; tb < t_stop; tb += ncb * CH) {
    p.t0 = tb;
    p.nt = std::min(ncb * CH, t_stop - tb);
    p.NCb = (p.nt + CH - 1) / CH;
    const bool first = tb == a->t0;
    p.has_init = first ? (a->init_state != nullptr) : 1;
    p.init = first ? a->init_state : carry;
    p.fin = carry;
    const hipError_t e = dispatch(p, st, bf, a->qk_dtype, a->v_dtype == DN_BF16);
    if (e != hipSuccess) return set_error(DN_E_LAUNCH, hipGetErrorString(e));
  }
  return DN_OK;
}
