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
// The MI355X design splits the work into two launches per token block so
// that only a 128x128-by-128x16 product sits on the sequential critical path.
// With Vnew = U - W S the reference's per-chunk update and output become
//     S_next = [same doc] diag(e^Lend) S + Pn S + Q,  Pn = -ke^T W,  Q = ke^T U
//     O      = X S + Oi,                              X = qe - M W,  Oi = M U
// so:
//   k_prepass (grid: one workgroup of 8 waves per (batch, exec head, chunk)
//       unit) fused prologue, Lambda, A and M on MFMA, T by blocked
//       substitution on fp32 MFMA, W, the chunk operators Pn and X, and
//       then, from the T, ke^T and M it still holds in LDS, U = T (w*v),
//       Q = ke^T U and Oi = M U (value_cols).
//   k_chain   (grid: 16-column tile x exec-head x batch, 8 waves)
//       the sequential scan over chunks with the fp32 state in VGPRs, and
//       each chunk's output O = X S_c + Oi from the same S_c fragments.
//
// Intermediates live in a caller-provided workspace sized for one token
// block, small enough to stay resident in the 256 MB Infinity Cache; every
// array is stored in the MFMA lane order of its consumer.
#include <mutex>

#include "dn_common.h"
#include "dn_host.h"

namespace dn {

constexpr int CH = 128;   // chunk size (gdn2.py:1869)
constexpr int KD = 128;   // key / value head dim (gdn2.py:1897)
constexpr int XP = 132;
constexpr int kMaxBlockChunks = 1024;   // chunks per token block (chain's LDS flag table)
   // fp32 LDS pitch (floats): conflict-free 16-lane column groups

// diag blocks whose in-block log2-decay span exceeds this use the
// overflow-free hierarchical path (e^{69} stays far inside the fp32 range)
constexpr float kDiagSafeLog2 = 100.f;

// ---------------------------------------------------------------------------
// gate activations (gdn2.py:38-47, 133-142, 1970-1974): g = -exp(min(g, 5)),
// b, w = sigmoid.  The sigmoid uses the hardware reciprocal (v_rcp_f32, 1 ulp):
// 1 + e^{-x} >= 1, and an infinite denominator gives exactly 0.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float sigmoid_fast(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }

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

// A segment id as two 32-bit words loaded without a branch, so the loads can
// be issued early (the value is only compared for equality).  int32 ids read
// their word twice.
// A segment id as its two 32-bit words; an int32 id repeats its one word in
// hi (no select on the loaded value, so nothing waits for the load until the
// ids are compared; equality is unchanged)
struct SegId {
  int32_t lo, hi;
  __device__ __forceinline__ bool operator!=(const SegId& o) const { return lo != o.lo || hi != o.hi; }
};
__device__ __forceinline__ SegId seg_raw(const PF& p, int b, int t) {
  const int64_t i = p.seg_batched ? (int64_t)b * p.L + t : (int64_t)t;
  const bool w64 = p.seg_dt == DT_I64;
  const int32_t* s32 = (const int32_t*)p.seg + (w64 ? 2 * i : i);
  return SegId{s32[0], s32[w64 ? 1 : 0]};
}

// v rows of one 32-column slab of execution head h, chunk c (row 16a + r16 of
// block a, fragment order, as loaded) and the write gate of those rows when it
// has one channel.  Issued apart from their use so a caller can put them in
// flight ahead of other work: vmcnt counts loads and stores in issue order, so
// the wait for these rows covers only what was issued before them.
template <class TV> struct VRows {
  Raw8<TV> v[8];
  float ws[8];
};

template <class TV>
__device__ __forceinline__ void v_rows_issue(const PF& p, int b, int h, int c, int col0, int l, VRows<TV>& r) {
  const int r16 = l & 15, q = l >> 4;
  const int tb = p.t0 + c * CH;
  const int t_end = min(p.t0 + p.nt, p.L);
  const int hv = p.gates_at_hv ? h : h * p.G + col0 / KD;
  const int hw = vgate_head(p, p.w_h, hv);
  const int cs = (col0 & ~31) % KD;
  auto row_bt = [&](int a) { return (int64_t)b * p.L + min(tb + 16 * a + r16, t_end - 1); };
  // (the w layout test sits outside the row loops: a branch between the
  // loads would make each row wait for the one before)
  if (p.w_c == 1) {
#pragma unroll
    for (int a = 0; a < 8; ++a) {
      const int64_t bt = row_bt(a);
      r.v[a].load((const TV*)p.v + (bt * p.Hv + hv) * KD + cs, q);
      r.ws[a] = ((const float*)p.w)[bt * p.w_h + hw];
    }
  } else {
#pragma unroll
    for (int a = 0; a < 8; ++a) {
      r.v[a].load((const TV*)p.v + (row_bt(a) * p.Hv + hv) * KD + cs, q);
      r.ws[a] = 0.f;
    }
  }
}

// (w*v)^T fragments of 16 NT value columns of execution head h, chunk c, from
// column col0 (rows = value column, k = token): Bwv[nt][s] covers columns
// col0 + 16nt .. + 15 and token slab s, from the rows r (v_rows_issue of the
// same columns).  Each 16-token block is transposed by an identity product
// into half of a slab (exact).
template <bool BF, class TV, int NT>
__device__ __forceinline__ void wv_frags(const PF& p, int b, int h, int c, int col0, int l, const VRows<TV>& r,
                                         typename Pol<BF>::F3 (&Bwv)[NT][4]) {
  using P = Pol<BF>;
  using F1 = typename P::F1;
  using F3 = typename P::F3;
  const int r16 = l & 15, q = l >> 4;
  const int tb = p.t0 + c * CH;
  const int t_end = min(p.t0 + p.nt, p.L);
  const int hv = p.gates_at_hv ? h : h * p.G + col0 / KD;
  const int hw = vgate_head(p, p.w_h, hv);
  const int h0 = NT == 2 ? 0 : (col0 >> 4) & 1;   // first 16-column half of the slab
  const int cs = (col0 & ~31) % KD;
  float ww[8][8];
  if (p.w_c == 1) {
#pragma unroll
    for (int a = 0; a < 8; ++a)
#pragma unroll
      for (int e = 0; e < 8; ++e) ww[a][e] = r.ws[a];
  } else {
#pragma unroll
    for (int a = 0; a < 8; ++a) {
      const int64_t bt = (int64_t)b * p.L + min(tb + 16 * a + r16, t_end - 1);
      row8<float>((const float*)p.w + (bt * p.w_h + hw) * p.w_c + cs, q, ww[a]);
    }
  }
  const F1 id0 = ident_frag<BF>(0, r16, q), id1 = ident_frag<BF>(1, r16, q);
#pragma unroll
  for (int a = 0; a < 8; ++a) {
    const bool valid = tb + 16 * a + r16 < t_end;
    float vv[8], x[8];
    r.v[a].to(vv);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float wg = p.fuse ? sigmoid_fast(ww[a][e]) : ww[a][e];
      x[e] = valid ? wg * vv[e] : 0.f;
    }
    const F3 fx = P::f3(x);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const bool second = nt + h0 == 1;
      f32x4 chi = zero4();
      mma(chi, P::hi(fx), second ? id1 : id0);
      // lane (c, q): column 16nt + c, tokens 16a + 4q + ii -> slab a/2, half a&1
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        if constexpr (BF) {
          Bwv[nt][a >> 1].hi.v[4 * (a & 1) + ii] = (bf16)chi[ii];
        } else {
          Bwv[nt][a >> 1].v[4 * (a & 1) + ii] = chi[ii];
        }
      }
      if constexpr (BF) {
        f32x4 clo = zero4();
        mma(clo, fx.lo, second ? id1 : id0);
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) Bwv[nt][a >> 1].lo.v[4 * (a & 1) + ii] = (bf16)clo[ii];
      }
    }
  }
}

// q, k and b * k of one token row in fragment order (slab s: elements
// 8s..8s+7), after the prologue: L2 normalisation (gdn2.py:1990-1996, the
// normalised q and k rounded back to the input type), the q scale, the b
// activation or clamp, and zeros for tokens past the end.
template <class TIn>
__device__ __forceinline__ void row_inputs(const PF& p, const Raw8<TIn> (&rq)[4], const Raw8<TIn> (&rk)[4],
                                           const Raw8<float> (&rb)[4], float b_scalar, bool valid, float (&qv)[32],
                                           float (&kv)[32], float (&bet)[32]) {
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    rq[s].to(qv + 8 * s);
    rk[s].to(kv + 8 * s);
  }
  if (p.b_c == 1) {
#pragma unroll
    for (int e = 0; e < 32; ++e) bet[e] = b_scalar;
  } else {
#pragma unroll
    for (int s = 0; s < 4; ++s) rb[s].to(bet + 8 * s);
  }
  float ssq = 0.f, ssk = 0.f;
#pragma unroll
  for (int e = 0; e < 32; ++e) { ssq += qv[e] * qv[e]; ssk += kv[e] * kv[e]; }
  ssq += __shfl_xor(ssq, 16); ssq += __shfl_xor(ssq, 32);
  ssk += __shfl_xor(ssk, 16); ssk += __shfl_xor(ssk, 32);
  if (p.fuse) {
    const float rq = rsqrtf(ssq + 1e-6f) , rk = rsqrtf(ssk + 1e-6f);
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      qv[e] = (qv[e] * rq) * p.scale;
      kv[e] = kv[e] * rk;
      bet[e] = sigmoid_fast(bet[e]);
    }
  } else if (p.l2norm) {
    const float rq = rsqrtf(ssq + 1e-6f), rk = rsqrtf(ssk + 1e-6f);
#pragma unroll
    for (int e = 0; e < 32; ++e) { qv[e] = round_as<TIn>((qv[e] * rq) * p.scale); kv[e] = round_as<TIn>(kv[e] * rk); }
  } else {
#pragma unroll
    for (int e = 0; e < 32; ++e) qv[e] = round_as<TIn>(qv[e] * p.scale);
  }
  if (p.guard && !p.fuse) {
#pragma unroll
    for (int e = 0; e < 32; ++e) bet[e] = fmaxf(bet[e], 0.f);
  }
#pragma unroll
  for (int e = 0; e < 32; ++e) {
    qv[e] = valid ? qv[e] : 0.f;
    kv[e] = valid ? kv[e] : 0.f;
    bet[e] = valid ? bet[e] * kv[e] : 0.f;
  }
}

// ===========================================================================
// Phases 1-3 of k_prepass for one decay and one b per (token, head) (the
// Gated DeltaNet form, chunk_gdn: gdn.py:66-110 broadcasts them over the key
// channels), precision "bf16" with bf16 q and k.  The per-channel machinery of
// the general phases collapses:
//   * Lambda is one cumulative sum per token (double-float, log2 units);
//   * with the normalised q and k exactly bf16 (they are rounded back to the
//     input type), the Gram matrices k k^T and q k^T are single bf16 MFMAs
//     with fp32 accumulation, and
//       A[i][j] = b_i e^{Lambda_i - Lambda_j} (k k^T)[i][j]   (i > j),
//       M[i][j] =     e^{Lambda_i - Lambda_j} (q k^T)[i][j]   (i >= j),
//     one exponential per pair, whose exponent is <= 0 for every unmasked
//     pair (no factorisation, no overflow path);
//   * (b k e^Lambda)^T, ke^T, qe and e^{Lambda_end} are per-row scalars times
//     the row.
// Results land where the general phases put them: A (fp32, row-major) in X,
// M (split, fragment-native) and the transposed row operands in the
// workspace; Y holds the q and k fragments until phase 4 takes it over.
// Barriers inside wait for LDS only, so the per-row stores drain behind the
// Gram products; the last one (a full __syncthreads) drains them before any
// wave reads another's rows back.
// ===========================================================================
template <class TIn>
__device__ __forceinline__ void prepass_scalar_gates(const PF& p, int b, int tb, int t_end, float g_tok,
                                                     const Raw8<TIn> (&rq)[4], const Raw8<TIn> (&rk)[4],
                                                     const Raw8<float> (&rb)[4], float b_scalar, const int* doc,
                                                     float* X, float* Y, bf16* g_Mh, bf16* g_Ml, bf16* g_be,
                                                     bf16* g_keh, bf16* g_kel, float* g_qe, float* g_dv) {
  using P = Pol<true>;
  using F1 = P::F1;
  using F3 = P::F3;
  using SS = Store<true>;
  __shared__ float lam_h[CH], lam_l[CH];   // Lambda (log2 units), double-float
  __shared__ float bet_s[CH];              // b per token (0 past the end)
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, r16 = l & 15, q = l >> 4;

  // ---- Lambda: inclusive scan of g over the chunk (waves 0 and 1) ----------
  float hi = 0.f, lo = 0.f;
  if (tid < CH) {
    float gv = fminf(g_tok, 0.f);   // _nonpositive (NaN -> 0)
    gv = fminf(gv, p.guard ? -1e-6f : 0.f);
    hi = (tb + tid < t_end) ? gv : 0.f;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float h2 = __shfl_up(hi, off), l2 = __shfl_up(lo, off);
      if (l >= off) {
        // error-free hi + h2 (TwoSum), the rounding error joins the low words
        const float sum = hi + h2;
        const float bb = sum - hi;
        lo += l2 + ((hi - (sum - bb)) + (h2 - bb));
        hi = sum;
      }
    }
    if (w == 0 && l == 63) { lam_h[63] = hi; lam_l[63] = lo; }
  }
  lds_barrier();
  if (tid < CH) {
    if (w == 1) {
      const float h2 = lam_h[63], l2 = lam_l[63];
      const float sum = hi + h2;
      const float bb = sum - hi;
      lo += l2 + ((hi - (sum - bb)) + (h2 - bb));
      hi = sum;
    }
  }
  lds_barrier();
  if (tid < CH) {
    const float ph = hi * kLog2e;
    lam_h[tid] = ph;
    lam_l[tid] = fmaf(hi, kLog2e, -ph) + lo * kLog2e;
  }
  lds_barrier();
  const float le_h = lam_h[CH - 1], le_l = lam_l[CH - 1];
  if (tid < KD) g_dv[tid] = fast_exp2(le_h + le_l);   // e^{Lambda_end}

  // ---- per-row operands of token block a = w --------------------------------
  bf16* Kf = reinterpret_cast<bf16*>(Y);   // k fragments [block][slab][lane][8]
  bf16* Qf = Kf + CH * KD;                 // q fragments
  {
    const int a = w;
    const int i = 16 * a + r16;
    const bool valid = tb + i < t_end;
    float qv[32], kv[32], bet[32];
    row_inputs<TIn>(p, rq, rk, rb, b_scalar, valid, qv, kv, bet);
    // b alone: b * k / k is not recoverable where k = 0, so take it again
    float bsc = p.b_c == 1 ? b_scalar : 0.f;
    if (p.guard) bsc = fmaxf(bsc, 0.f);
    if (q == 0) bet_s[i] = valid ? bsc : 0.f;
    const bool first = doc[i] == 0;
    const bool last = doc[i] == doc[CH - 1];
    const float li_h = lam_h[i], li_l = lam_l[i];
    const float eL = fast_exp2(li_h + li_l);                    // e^{Lambda_i} <= 1
    const float eK = fast_exp2((le_h - li_h) + (le_l - li_l));  // e^{Lambda_end - Lambda_i} <= 1
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      float bt[8], kt[8], qe[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        bt[e] = first ? bet[8 * s + e] * eL : 0.f;
        kt[e] = last ? kv[8 * s + e] * eK : 0.f;
        qe[e] = first ? qv[8 * s + e] * eL : 0.f;
      }
      Store<false>::st8(g_qe + fofs(a, s, l), qe);
      // (b k e^Lambda)^T and ke^T in fragment layout (row = key, k = token)
      const F1 fbt = P::f1(bt);
      const F3 fkt = P::f3(kt);
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const F1 id = ident_frag<true>(hf, r16, q);
        f32x4 cb = zero4(), chi = zero4(), clo = zero4();
        mma(cb, fbt, id);
        mma(chi, fkt.hi, id);
        mma(clo, fkt.lo, id);
        const int o = fofs(2 * s + hf, a >> 1, l) + 4 * (a & 1);
        const float xb[4] = {cb[0], cb[1], cb[2], cb[3]};
        const float xh[4] = {chi[0], chi[1], chi[2], chi[3]};
        const float xl[4] = {clo[0], clo[1], clo[2], clo[3]};
        SS::st4(g_be + o, xb);
        SS::st4(g_keh + o, xh);
        SS::st4(g_kel + o, xl);
      }
      // the normalised rows are bf16 values: their fragments are exact
      SS::st8(Kf + fofs(a, s, l), kv + 8 * s);
      SS::st8(Qf + fofs(a, s, l), qv + 8 * s);
    }
  }
  lds_barrier();

  // ---- A and M tiles (a, bb), bb <= a: 36 tiles dealt round-robin ------------
  for (int t = w; t < 36; t += 8) {
    int a = 0;
    while ((a + 1) * (a + 2) / 2 <= t) ++a;
    const int bb = t - a * (a + 1) / 2;
    f32x4 gk = zero4(), gq = zero4();
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const F1 ka = SS::fa(Kf + fofs(a, s, l));
      const F1 kb = SS::fa(Kf + fofs(bb, s, l));
      const F1 qa = SS::fa(Qf + fofs(a, s, l));
      mma(gk, ka, kb);   // (k k^T)[16a + 4q + ii][16bb + r16]
      mma(gq, kb, qa);   // (q k^T)[16a + r16][16bb + 4q + ii]
    }
    float mv[4];
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      {
        const int i = 16 * a + 4 * q + ii, j = 16 * bb + r16;
        const float d = (lam_h[i] - lam_h[j]) + (lam_l[i] - lam_l[j]);
        const bool on = i > j && doc[i] == doc[j];
        X[i * XP + j] = on ? bet_s[i] * fast_exp2(fminf(d, 0.f)) * gk[ii] : 0.f;
        if (bb == a && (a & 1) == 0) X[i * XP + j + 16] = 0.f;
      }
      {
        const int i = 16 * a + r16, j = 16 * bb + 4 * q + ii;
        const float d = (lam_h[i] - lam_h[j]) + (lam_l[i] - lam_l[j]);
        const bool on = i >= j && doc[i] == doc[j];
        mv[ii] = on ? fast_exp2(fminf(d, 0.f)) * gq[ii] : 0.f;
      }
    }
    const int mo = fofs(a, bb >> 1, l) + 4 * (bb & 1);
    SS::st4s(g_Mh + mo, g_Ml + mo, mv);
    if (bb == a && (a & 1) == 0) {
      const float z[4] = {0.f, 0.f, 0.f, 0.f};
      SS::st4s(g_Mh + mo + 4, g_Ml + mo + 4, z);
    }
  }
  __syncthreads();
}

// ===========================================================================
// k_prepass: everything per chunk that does not depend on the values (one
// workgroup of 8 waves per (chunk, execution head, batch); wave w owns token
// block w in the per-row phases and key tile w in phase 5): chunk flags,
// Lambda, A and M, T = (I + A)^-1, W = T (b k e^Lambda), Pn = -ke^T W and
// X = qe - M W; then U, Q and (M U)^T of every value column (value_cols).
//
// Lambda is kept block-local: X[i] = sum of g over the 16-token block of i up
// to and including i (log2 units, double-float hi in X / lo in Y), so a
// difference of two Lambdas is never the difference of two large cumulative
// sums (no fp32 cancellation after a strongly decayed stretch).  Cross-block
// factors come from the per-block totals (sums of the totals before / after
// block a, kept as the exponentials Ea / Sa).
//
// Products whose result feeds another kernel are computed transposed where
// that puts the result directly in its consumer's fragment layout (M^T, Pn^T,
// X^T); (b k e^Lambda)^T and ke^T are transposed by an identity product.
// ===========================================================================
template <bool BF, class TV, int NT>
__device__ __forceinline__ void value_cols(const PF& p, int b, int h, int c, int col0, int l, const VRows<TV>& vr,
                                           const typename Store<BF>::ST* g_T, const typename Store<BF>::ST* g_keh,
                                           const typename Store<BF>::ST* g_kel, const typename Store<BF>::ST* g_Mh,
                                           const typename Store<BF>::ST* g_Ml);

template <bool BF, class TIn, class TV, bool SC>
__global__ __launch_bounds__(512) void k_prepass(const PF p) {
  using P = Pol<BF>;
  using F1 = typename P::F1;
  using F3 = typename P::F3;
  using SS = Store<BF>;
  using ST = typename SS::ST;
  constexpr int YP = 132;
  __shared__ float X[CH * XP];        // Lambda hi -> A -> T (fp32)
  __shared__ float Y[CH * YP];        // Lambda lo -> Kc -> T fragment-native (ST)
  __shared__ float Ftab[8 * KD];      // e^{total of block b}
  __shared__ float Mid0[8 * KD];      // e^{g at the first token of block a}
  __shared__ float Ea[8 * KD];        // e^{Lambda at the first token of block a} (chunk-global)
  __shared__ float Sa[8 * KD];        // e^{sum of the totals of blocks > a}
  __shared__ float Fa[8 * KD];        // e^{Lambda(last) - Lambda(first token) of block a}
  __shared__ float Gt[8 * KD];        // e^{Lambda(first token of block a) - Lambda(row 64)}
  __shared__ int doc[CH];
  __shared__ int unsafe_part[2][8];   // per 64-channel half: block needs the hierarchical path
  __shared__ int wide_part[2];        // per 64-channel half: the chunk-reference path is unsafe

  const int tid = threadIdx.x;
  // (the wave index as a scalar: loops and tile indices over waves stay in
  // scalar registers, with no per-lane masks)
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, r16 = l & 15, q = l >> 4;
  const int units = p.B * p.Hx * p.NCb;
  // chunk unit: XCD-aware remap (the hardware deals linear block ids to the 8
  // XCDs round-robin; consecutive chunks of a head share one XCD's L2)
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
  const int64_t uf = u * (CH * KD);   // one 128 x 128 fragment-native array per unit
  const int hk = p.gates_at_hv ? h / p.G : h;

  ST* g_Pn = (ST*)p.PnA + uf;
  ST* g_Xh = (ST*)p.XAh + uf;
  ST* g_Xl = (ST*)p.XAl + uf;
  ST* g_be = (ST*)p.BeB + uf;
  ST* g_keh = (ST*)p.KeBh + uf;
  ST* g_kel = (ST*)p.KeBl + uf;
  ST* g_Mh = (ST*)p.MAh + uf;
  ST* g_Ml = (ST*)p.MAl + uf;
  float* g_qe = p.QeA + uf;
  float* g_dv = p.dvec + u * KD;

  // Global loads are issued up front, in the order their values are needed
  // (the vector-memory counter drains in order, so a load is only ever waited
  // for together with the loads issued before it): segment ids (phase 0),
  // gates g (phase 1), then the q, k, b rows of this wave's token block
  // (phase 2), whose latency then overlaps phases 0 and 1.
  // (every lane loads, under wave-uniform conditions only, so no value is
  // consumed inside a divergent branch before it is needed)
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
  const int g_part = tid >> 7;   // phase 1: 4 parts of 32 tokens, channel tid & 127
  float gl[SC ? 1 : 32];
  if constexpr (SC) {
    // one decay per token: thread t < 128 loads token t's (clamped to the last valid)
    gl[0] = 0.f;
    if (tid < CH) {
      const int hg = kgate_head(p, p.g_h, h);
      gl[0] = ((const float*)p.g)[((int64_t)b * p.L + min(tb + tid, t_end - 1)) * p.g_h + hg];
    }
  } else {
    const int kap = tid & 127;
    const int hg = kgate_head(p, p.g_h, h);
    const int tload = min(tb + 32 * g_part, t_end - 1);
    const int nload = t_end - tload;   // >= 1
    const int gstride = p.g_h * p.g_c;
    const float* gp = (const float*)p.g + (((int64_t)b * p.L + tload) * p.g_h + hg) * p.g_c + (p.g_c == 1 ? 0 : kap);
    // out-of-range tokens read the last valid token and are zeroed in phase 1
#pragma unroll
    for (int i = 0; i < 32; ++i) gl[i] = gp[min(i, nload - 1) * gstride];
  }
  const int hbg = kgate_head(p, p.b_h, h);
  Raw8<TIn> rq[4], rk[4];
  Raw8<float> rb[4];
  float b_scalar = 0.f;
  {
    const int t = tb + 16 * w + r16;
    const int tt = t < t_end ? t : tb;
    const TIn* qp = (const TIn*)p.q + (((int64_t)b * p.L + tt) * p.Hk + hk) * KD;
    const TIn* kp = (const TIn*)p.k + (((int64_t)b * p.L + tt) * p.Hk + hk) * KD;
    const float* bp = (const float*)p.b + (((int64_t)b * p.L + tt) * p.b_h + hbg) * p.b_c;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      rq[s].load(qp + 32 * s, q);
      rk[s].load(kp + 32 * s, q);
    }
    if (p.b_c == 1) {
      b_scalar = bp[0];
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) rb[s].load(bp + 32 * s, q);
    }
  }
  // first use of the segment ids: only now, after every entry load is issued
  // (an empty asm that "updates" them keeps the compiler from comparing them
  // earlier, which would wait before the later loads are even issued)
  asm volatile("" : "+v"(sg_t.lo), "+v"(sg_t.hi), "+v"(sg_tp.lo), "+v"(sg_tp.hi));
  asm volatile("" : "+v"(sg_0.lo), "+v"(sg_0.hi), "+v"(sg_a.lo), "+v"(sg_a.hi), "+v"(sg_b.lo), "+v"(sg_b.hi));

  // ---- phase 0: in-chunk document index (segment canonicalisation) -------
  // doc[i] = number of segment starts among tokens 1..i: a wave ballot and a
  // popcount per token (waves 0 and 1 hold tokens 0..127), wave 1 adding
  // wave 0's total
  {
    __shared__ int starts0;
    const bool st = tid < CH && tid > 0 && p.seg != nullptr && (sg_t != sg_tp);
    const uint64_t bal = __ballot(st);
    const int upto = __popcll(bal & ((2ull << l) - 1ull));   // lanes 0..l (l = 63: all)
    if (tid == 0) starts0 = __popcll(bal);
    __syncthreads();
    if (tid < CH) doc[tid] = upto + (w == 1 ? starts0 : 0);
    __syncthreads();
  }
  if (tid == 0 && h == 0) {
    int is_new;
    if (tb == 0) {
      if (p.has_init) {
        is_new = 0;
        // initial_state_segment_id is int32; a wider first id differs from it
        // when its high word is not the sign extension of its low word
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
    p.flags[((int64_t)b * p.NCb + c) * 2 + 1] = (doc[CH - 1] == 0);
  }

  if constexpr (SC) {
    prepass_scalar_gates<TIn>(p, b, tb, t_end, gl[0], rq, rk, rb, b_scalar, doc, X, Y, g_Mh, g_Ml, g_be, g_keh,
                              g_kel, g_qe, g_dv);
  } else {
  // ---- phase 1: block-local Lambda (double-float: X = hi, Y = lo), totals --
  {
    const int kap = tid & 127, part = g_part;
    const int nvalid = t_end - (tb + 32 * part);   // tokens of this part in range (may be <= 0)
    if (p.fuse) {
#pragma unroll
      for (int i = 0; i < 32; ++i) gl[i] = -__expf(fminf(gl[i], 5.f));
    } else {
#pragma unroll
      for (int i = 0; i < 32; ++i) gl[i] = fminf(gl[i], 0.f);  // _nonpositive (NaN -> 0)
    }
    const float gmax = p.guard ? -1e-6f : 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) gl[i] = (i < nvalid) ? fminf(gl[i], gmax) : 0.f;
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
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
        const int row = 32 * part + 16 * blk + j;
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
    float acc = 0.f, lg[8];
#pragma unroll
    for (int a = 0; a < 8; ++a) {
      const float lsa = X[(16 * a) * XP + tid] + Y[(16 * a) * XP + tid];
      lg[a] = acc + lsa;   // chunk-global Lambda at the first token of block a
      Ea[a * KD + tid] = fast_exp2(lg[a]);
      acc += tot[a];
    }
    g_dv[tid] = fast_exp2(acc);   // e^{Lambda_end}
    // chunk reference row 64: every off-diagonal A / M entry factors as
    // (row i: e^{Lambda_i - Lambda_64}) (column j: e^{Lambda_64 - Lambda_j}),
    // both within 2^{+-100} when the spans on either side of row 64 are
    bool wide = (lg[0] - lg[4] > kDiagSafeLog2) || (lg[4] - acc > kDiagSafeLog2);
#pragma unroll
    for (int a = 0; a < 8; ++a) Gt[a * KD + tid] = fast_exp2(lg[a] - lg[4]);
    acc = 0.f;
#pragma unroll
    for (int a = 7; a >= 0; --a) { Sa[a * KD + tid] = fast_exp2(acc); acc += tot[a]; }
#pragma unroll
    for (int a = 0; a < 8; ++a) {
      Ftab[a * KD + tid] = fast_exp2(tot[a]);
      Mid0[a * KD + tid] = fast_exp2(X[(16 * a) * XP + tid] + Y[(16 * a) * XP + tid]);
      // span of the block after its first token: Lambda(sa) - Lambda(ea) >= 0
      const int sa = 16 * a, ea = sa + 15;
      const float span = (X[sa * XP + tid] - X[ea * XP + tid]) + (Y[sa * XP + tid] - Y[ea * XP + tid]);
      Fa[a * KD + tid] = fast_exp2(-span);
      const bool un = __any(span > kDiagSafeLog2);
      if (l == 0) unsafe_part[w][a] = un;
      wide = wide || un;
    }
    wide = __any(wide);
    if (l == 0) wide_part[w] = wide;
  }
  __syncthreads();
  // no block needs the hierarchical path and the chunk reference is safe:
  // phase 2 leaves the column factors of every block as split fragments in
  // Y, and phase 3 is MFMA products of stored fragments only
  const bool chunk_ref = __builtin_amdgcn_readfirstlane(!(wide_part[0] | wide_part[1]));

  // ---- phase 2: per-row quantities, diagonal A/M blocks --------------------
  F3 Rf[1][4], Qf[1][4];
  f32x4 Adiag[1];
#pragma unroll
  for (int bi = 0; bi < 1; ++bi) {
    const int a = w;
    const int i = 16 * a + r16;
    const int t = tb + i;
    const bool valid = t < t_end;
    float qv[32], kv[32], bet[32];
    row_inputs<TIn>(p, rq, rk, rb, b_scalar, valid, qv, kv, bet);
    const bool first = doc[i] == 0;
    const bool last = doc[i] == doc[CH - 1];
    const bool blk_unsafe = unsafe_part[0][a] | unsafe_part[1][a];
    // accA: A tile (lane = column token); accM: M^T tile (lane = row token)
    f32x4 accA = zero4(), accM = zero4();
    float dq = 0.f;
#pragma unroll
    for (int e = 0; e < 32; ++e) dq += qv[e] * kv[e];
    dq += __shfl_xor(dq, 16);
    dq += __shfl_xor(dq, 32);
    // Blocks with a large in-block decay span take the hierarchical path
    // first, while the slab loop's fragments are not yet live.
    if (blk_unsafe) {
      // Overflow-free hierarchical factorisation: the pair (i, j) is split at
      // the highest bit where the in-block indices differ; rows above and
      // columns below the split point are scaled toward it, so every
      // exponent is <= 0.  (accM holds the transposed tile, as above.)
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
          P::m33(tM, fb, P::f3(xm));
        }
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          const int il = 4 * q + ii;
          const int hb = 31 - __builtin_clz((il ^ r16) | 1);  // il == r16 selects nothing
          if (il > r16 && hb == hl) accA[ii] = tA[ii];
          if (r16 > il && hb == hl) accM[ii] = tM[ii];
        }
      }
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
        if (4 * q + ii == r16) accM[ii] = dq;
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      float lam[8], lsa[8], laml[8], lsal[8], ea[8], sa[8];
      row8<float>(&X[i * XP + 32 * s], q, lam);
      row8<float>(&X[(16 * a) * XP + 32 * s], q, lsa);
      row8<float>(&Y[i * XP + 32 * s], q, laml);
      row8<float>(&Y[(16 * a) * XP + 32 * s], q, lsal);
      row8<float>(&Ea[a * KD + 32 * s], q, ea);
      row8<float>(&Sa[a * KD + 32 * s], q, sa);
      float rA[8], rM[8], bd[8], kc[8], qe[8], bt[8], kt[8];
      if (!blk_unsafe) {
        // every factor within 2^{+-100}: the exponentials of the row's
        // decay relative to the block's first token and their products
        float fa[8];
        row8<float>(&Fa[a * KD + 32 * s], q, fa);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float qh = qv[8 * s + e], kh = kv[8 * s + e], be = bet[8 * s + e];
          const float d_i_sa = (lam[e] - lsa[e]) + (laml[e] - lsal[e]);   // <= 0
          const float er = fast_exp2(d_i_sa);
          const float rr = fast_exp2(-d_i_sa);
          rA[e] = be * er;
          rM[e] = qh * er;
          const float ekc = fa[e] * rr;                 // e^{Lambda(ea) - Lambda(i)}
          kc[e] = kh * ekc;
          const float eL = ea[e] * er;                  // e^{Lambda(i)} (chunk-global)
          bt[e] = first ? be * eL : 0.f;
          kt[e] = last ? kc[e] * sa[e] : 0.f;
          bd[e] = kh * rr;
          qe[e] = first ? qh * eL : 0.f;
        }
      } else {
        float ta[8], tal[8];
        row8<float>(&X[(16 * a + 15) * XP + 32 * s], q, ta);
        row8<float>(&Y[(16 * a + 15) * XP + 32 * s], q, tal);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float qh = qv[8 * s + e], kh = kv[8 * s + e], be = bet[8 * s + e];
          const float d_i_sa = (lam[e] - lsa[e]) + (laml[e] - lsal[e]);   // <= 0
          const float d_ea_i = (ta[e] - lam[e]) + (tal[e] - laml[e]);     // <= 0
          const float er = fast_exp2(d_i_sa);
          rA[e] = be * er;
          rM[e] = qh * er;
          const float ekc = fast_exp2(d_ea_i);
          kc[e] = kh * ekc;
          const float eL = ea[e] * er;
          bt[e] = first ? be * eL : 0.f;
          kt[e] = last ? kh * ekc * sa[e] : 0.f;
          bd[e] = 0.f;   // unused: the hierarchical path formed this block's A and M
          qe[e] = first ? qh * eL : 0.f;
        }
      }
      Store<false>::st8(g_qe + fofs(a, s, l), qe);
      {
        // (b k e^Lambda)^T and ke^T in fragment layout (row = key, k = token)
        const F1 fbt = P::f1(bt);
        const F3 fkt = P::f3(kt);
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          const F1 id = ident_frag<BF>(hf, r16, q);
          f32x4 cb = zero4(), chi = zero4();
          mma(cb, fbt, id);
          mma(chi, P::hi(fkt), id);
          const int o = fofs(2 * s + hf, a >> 1, l) + 4 * (a & 1);
          const float xb[4] = {cb[0], cb[1], cb[2], cb[3]};
          const float xh[4] = {chi[0], chi[1], chi[2], chi[3]};
          SS::st4(g_be + o, xb);
          SS::st4(g_keh + o, xh);
          if constexpr (BF) {
            f32x4 clo = zero4();
            mma(clo, fkt.lo, id);
            const float xl[4] = {clo[0], clo[1], clo[2], clo[3]};
            SS::st4(g_kel + o, xl);
          }
        }
      }
      if (chunk_ref) {
        // rows relative to row 64 instead of the block's first token
        float gt[8];
        row8<float>(&Gt[a * KD + 32 * s], q, gt);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          rA[e] *= gt[e];
          rM[e] *= gt[e];
          bd[e] *= __builtin_amdgcn_rcpf(gt[e]);
        }
      }
      Rf[bi][s] = P::f3(rA);
      Qf[bi][s] = P::f3(rM);
      if (!blk_unsafe) {
        // A_aa, M_aa = (R, Qr) (k e^{Lambda_ref - Lambda})^T: every factor stays
        // within 2^{+-100} of 1, so the factorisation cannot overflow.
        const F3 fb = P::f3(bd);
        P::m33(accA, Rf[bi][s], fb);
        P::m33(accM, fb, Qf[bi][s]);
        if (chunk_ref) {
          // the column factors replace this slab's 16 rows x 32 columns of
          // Lambda low words (2 KB, once all lanes of the wave have read
          // them) as the split fragment of lane l: row l / 4, 32 bytes at
          // (l % 4) * 32 of the slab's 128 bytes in that row
          ST* fp = reinterpret_cast<ST*>(&Y[(16 * a + (l >> 2)) * YP + 32 * s]) + (l & 3) * (32 / sizeof(ST));
          SS::stf(fp, P::hi(fb));
          if constexpr (BF) SS::stf(fp + 8, fb.lo);
        }
      }
      if (!chunk_ref) {
        // Kc replaces this slab of the row's Lambda low words once all lanes
        // of the wave have read it (the other slabs' columns are untouched)
        st4<float>(&Y[i * YP + 32 * s + 4 * q], kc);
        st4<float>(&Y[i * YP + 32 * s + 16 + 4 * q], kc + 4);
      }
    }
    // diagonal blocks: A (row-major, LDS) and M (fragment-native, rows = token)
    float mv[4];
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const int il = 4 * q + ii, ia = 16 * a + il, ja = 16 * a + r16;
      const bool same = doc[ia] == doc[ja];
      Adiag[bi][ii] = (il > r16 && same) ? accA[ii] : 0.f;   // A[ia][ja]
      mv[ii] = (r16 >= il && same) ? accM[ii] : 0.f;          // M[ja][ia]
    }
    const int mo = fofs(a, a >> 1, l) + 4 * (a & 1);
    SS::st4s(g_Mh + mo, g_Ml + mo, mv);
    if ((a & 1) == 0) {
      const float z[4] = {0.f, 0.f, 0.f, 0.f};
      SS::st4s(g_Mh + mo + 4, g_Ml + mo + 4, z);
    }
  }
  __syncthreads();

  // ---- phase 3: off-diagonal A/M blocks (X becomes A) -----------------------
  // Block a has a pairs (a, bb < a).  Blocks 4..7 keep the pairs with
  // bb >= lo(a) = 1, 2, 3, 3 and hand the others to wave 7 - a, whose own
  // block has 7 - a pairs, so no wave computes more than 4.  The R / Q
  // fragments of blocks 4..7 reach those waves through X, which holds nothing
  // live between phases 2 and 4: every wave keeps its A tiles in registers
  // until all pairs are done and writes them to X afterwards.
  {
    constexpr int RQA = 2048;                       // elements per fragment array
    constexpr int RQB = (BF ? 4 : 2) * RQA;         // per block: R hi, (R lo,) Q hi, (Q lo)
    ST* rq_s = reinterpret_cast<ST*>(X);
    auto rq_ptr = [&](int a, int which, bool lo) -> ST* {   // which: 0 = R, 1 = Q
      return rq_s + (a - 4) * RQB + (BF ? (2 * which + (lo ? 1 : 0)) : which) * RQA;
    };
    if (w >= 4) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int o = (s * 64 + l) * 8;
        SS::stf(rq_ptr(w, 0, false) + o, P::hi(Rf[0][s]));
        SS::stf(rq_ptr(w, 1, false) + o, P::hi(Qf[0][s]));
        if constexpr (BF) {
          SS::stf(rq_ptr(w, 0, true) + o, Rf[0][s].lo);
          SS::stf(rq_ptr(w, 1, true) + o, Qf[0][s].lo);
        }
      }
    }
    __syncthreads();
    auto lo_of = [](int a) { return a < 4 ? 0 : (a == 4 ? 1 : (a == 5 ? 2 : 3)); };
    f32x4 Ap[4];
    int pa[4], pb[4];
    int np = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) { Ap[k] = zero4(); pa[k] = 0; pb[k] = 0; }
    // one pair's A tile (rows of block a) and M^T tile, masked by document
    auto pair_out = [&](int a, int bb, f32x4 accA, const f32x4& accM) {
      float mv[4];
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int ia = 16 * a + 4 * q + ii, jb = 16 * bb + r16;
        accA[ii] = (doc[ia] == doc[jb]) ? accA[ii] : 0.f;
        mv[ii] = (doc[16 * a + r16] == doc[16 * bb + 4 * q + ii]) ? accM[ii] : 0.f;
      }
      const int mo = fofs(a, bb >> 1, l) + 4 * (bb & 1);
      SS::st4s(g_Mh + mo, g_Ml + mo, mv);
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (np == k) { Ap[k] = accA; pa[k] = a; pb[k] = bb; }
      ++np;
    };
    auto pairs_ref = [&](int a, const F3 (&RF)[4], const F3 (&QF)[4], int bb_hi, int bb_lo) {
      auto ld_fb = [&](int bb, F3 (&fb)[4]) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const ST* fp = reinterpret_cast<const ST*>(&Y[(16 * bb + (l >> 2)) * YP + 32 * s]) + (l & 3) * (32 / sizeof(ST));
          if constexpr (BF) {
            fb[s].hi = SS::fa(fp);
            fb[s].lo = SS::fa(fp + 8);
          } else {
            fb[s] = SS::fa(fp);
          }
        }
      };
      F3 fb[4];
      ld_fb(bb_hi, fb);
      for (int bb = bb_hi; bb >= bb_lo; --bb) {
        // two accumulators per tile (leading and correction products) halve
        // the dependent MFMA chains
        f32x4 accA = zero4(), accM = zero4(), accA2 = zero4(), accM2 = zero4();
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          if constexpr (BF) {
            mma(accA, RF[s].hi, fb[s].hi);   // A[16a + 4q + ii][16bb + r16]
            mma(accM, fb[s].hi, QF[s].hi);   // M[16a + r16][16bb + 4q + ii]
            mma(accA2, RF[s].hi, fb[s].lo);
            mma(accM2, fb[s].hi, QF[s].lo);
            mma(accA2, RF[s].lo, fb[s].hi);
            mma(accM2, fb[s].lo, QF[s].hi);
          } else {
            P::m33(s & 1 ? accA2 : accA, RF[s], fb[s]);
            P::m33(s & 1 ? accM2 : accM, fb[s], QF[s]);
          }
        }
        if (bb > bb_lo) ld_fb(bb - 1, fb);
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) { accA[ii] += accA2[ii]; accM[ii] += accM2[ii]; }
        pair_out(a, bb, accA, accM);
      }
    };
    auto pairs = [&](int a, const F3 (&RF)[4], const F3 (&QF)[4], int bb_hi, int bb_lo) {
      if (chunk_ref) {
        pairs_ref(a, RF, QF, bb_hi, bb_lo);
        return;
      }
      float mloc[32];
#pragma unroll
      for (int s = 0; s < 4; ++s) row8<float>(&Mid0[a * KD + 32 * s], q, mloc + 8 * s);
      for (int b2 = a - 1; b2 > bb_hi; --b2) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          float f[8];
          row8<float>(&Ftab[b2 * KD + 32 * s], q, f);
#pragma unroll
          for (int e = 0; e < 8; ++e) mloc[8 * s + e] *= f[e];
        }
      }
      for (int bb = bb_hi; bb >= bb_lo; --bb) {
        f32x4 accA = zero4(), accM = zero4();
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          float x[8];
          row8<float>(&Y[(16 * bb + r16) * YP + 32 * s], q, x);
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] *= mloc[8 * s + e];
          const F3 fb = P::f3(x);
          P::m33(accA, RF[s], fb);   // A[16a + 4q + ii][16bb + r16]
          P::m33(accM, fb, QF[s]);   // M[16a + r16][16bb + 4q + ii]
        }
        pair_out(a, bb, accA, accM);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          float f[8];
          row8<float>(&Ftab[bb * KD + 32 * s], q, f);
#pragma unroll
          for (int e = 0; e < 8; ++e) mloc[8 * s + e] *= f[e];
        }
      }
    };
    pairs(w, Rf[0], Qf[0], w - 1, lo_of(w));
    if (w < 4) {
      const int a1 = 7 - w;
      F3 RF[4], QF[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int o = (s * 64 + l) * 8;
        RF[s] = SS::fa3(rq_ptr(a1, 0, false) + o, rq_ptr(a1, 0, true) + o);
        QF[s] = SS::fa3(rq_ptr(a1, 1, false) + o, rq_ptr(a1, 1, true) + o);
      }
      pairs(a1, RF, QF, lo_of(a1) - 1, 0);
    }
    __syncthreads();
    // A tiles of this wave's pairs and of its own diagonal block
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (k < np) {
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) X[(16 * pa[k] + 4 * q + ii) * XP + 16 * pb[k] + r16] = Ap[k][ii];
      }
    }
    {
      const int a = w;
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int ia = 16 * a + 4 * q + ii;
        X[ia * XP + 16 * a + r16] = Adiag[0][ii];
        if ((a & 1) == 0) X[ia * XP + 16 * a + 16 + r16] = 0.f;
      }
    }
  }
  __syncthreads();

  }

  // M (and, in bf16 mode, the high words of ke^T) are staged into LDS for
  // phase 5 once T no longer needs it; their loads are issued here so they
  // overlap the substitution.  16 bytes per load, 4 per array and thread.
  constexpr bool kStageKe = BF;
  using V16 = f32x4;
  V16 st_mh[4], st_ml[4], st_ke[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int o = (tid + 512 * j) * (16 / (int)sizeof(ST));   // element offset of chunk
    st_mh[j] = *reinterpret_cast<const V16*>(g_Mh + o);
    if constexpr (BF) st_ml[j] = *reinterpret_cast<const V16*>(g_Ml + o);
    if constexpr (kStageKe) st_ke[j] = *reinterpret_cast<const V16*>(g_keh + o);
  }

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
    // and transposed (Tt = Y, free during this phase: row 16a + r16 holds
    // column r16 of the block), the B operand layout of the steps below
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4)
      *reinterpret_cast<f32x4*>(&Y[(16 * a + r16) * YP + 16 * a + 4 * i4]) =
          f32x4{tc[4 * i4], tc[4 * i4 + 1], tc[4 * i4 + 2], tc[4 * i4 + 3]};
  }
  __syncthreads();
  // Block row a: T[a][bt] = -D_a sum_{cc = bt}^{a-1} A[a][cc] T[cc][bt], by
  // wave bt.  Each 16x16x16 product runs as 4 steps of the 16x16x4 fp32
  // MFMA with lane (r, q) holding reduction index 4q + kk at step kk, so a
  // lane's A operand (row of A) and B operand (row of T^T, kept in Y) are
  // one 16-byte LDS read each; all of a step's reads are issued before its
  // MFMAs, and the sum runs in two accumulation chains.
  float* Tt = Y;
  for (int a = 1; a < 8; ++a) {
    const int bt = w;
    f32x4 res = zero4();
    if (bt < a) {
      f32x4 Ar[7], Br[7];
#pragma unroll
      for (int cc = 0; cc < 7; ++cc) {
        if (cc >= bt && cc < a) {
          Ar[cc] = *reinterpret_cast<const f32x4*>(&X[(16 * a + r16) * XP + 16 * cc + 4 * q]);
          Br[cc] = *reinterpret_cast<const f32x4*>(&Tt[(16 * bt + r16) * YP + 16 * cc + 4 * q]);
        }
      }
      const f32x4 Dr = *reinterpret_cast<const f32x4*>(&X[(16 * a + r16) * XP + 16 * a + 4 * q]);
      f32x4 acc0 = zero4(), acc1 = zero4();
#pragma unroll
      for (int cc = 0; cc < 7; ++cc) {
        if (cc >= bt && cc < a) {
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) {
            if (cc & 1) acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(Ar[cc][kk], Br[cc][kk], acc1, 0, 0, 0);
            else acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(Ar[cc][kk], Br[cc][kk], acc0, 0, 0, 0);
          }
        }
      }
      f32x4 acc;
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) acc[ii] = acc0[ii] + acc1[ii];
      // lane (j, q) holds P[4q + ii][j]: the B operand of step kk is acc[kk]
      f32x4 r = zero4();
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) r = __builtin_amdgcn_mfma_f32_16x16x4f32(Dr[kk], acc[kk], r, 0, 0, 0);
      res = -r;
    }
    __syncthreads();
    if (bt < a) {
      // lane (j, q) holds T[16a + 4q + ii][16bt + j]
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) X[(16 * a + 4 * q + ii) * XP + 16 * bt + r16] = res[ii];
      *reinterpret_cast<f32x4*>(&Tt[(16 * bt + r16) * YP + 16 * a + 4 * q]) = res;
    }
    __syncthreads();
  }
  // T in fragment-native layout in Y (LDS), for W and the value columns.  In
  // bf16 mode its low words go after it, where ke^T is staged once W is formed.
  ST* Ts = reinterpret_cast<ST*>(Y);
  ST* Tl = Ts + CH * KD;
  F1 Bbe[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) Bbe[s] = SS::fa(g_be + fofs(w, s, l));
  for (int idx = w; idx < 32; idx += 8) {
    const int rt = idx >> 2, s = idx & 3;
    if (s > (rt >> 1)) continue;
    float x[8];
    row8<float>(&X[(16 * rt + r16) * XP + 32 * s], q, x);
    if constexpr (BF) SS::st8s(Ts + fofs(rt, s, l), Tl + fofs(rt, s, l), x);
    else SS::st8(Ts + fofs(rt, s, l), x);
  }
  __syncthreads();
  // ---- W = T be (key tile w) -------------------------------------------------
  // In bf16 mode T enters as high and low words: with nearly repeated keys
  // and b near 1, T is close to I minus a unit subdiagonal and W = T be
  // cancels to a small remainder, which a bf16-rounded T would leave with
  // 2^-9 / (1 - b) relative error (identical keys, b = 0.993: 7e-2 of the
  // output against 9e-3 with T split).
  f32x4 Wc[8];
#pragma unroll
  for (int rt = 0; rt < 8; ++rt) Wc[rt] = zero4();
#pragma unroll
  for (int rt = 0; rt < 8; ++rt) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (s <= rt / 2) {
        P::m11(Wc[rt], SS::fa(Ts + fofs(rt, s, l)), Bbe[s]);
        if constexpr (BF) P::m11(Wc[rt], SS::fa(Tl + fofs(rt, s, l)), Bbe[s]);
      }
    }
  }
  if constexpr (BF) __syncthreads();   // T's low words are read: ke^T takes their place
  // X (T in fp32) is free now: M high / low words there, ke^T high words
  // after T in Y (bf16 mode)
  ST* Mh_s = reinterpret_cast<ST*>(X);
  ST* Ml_s = BF ? Mh_s + CH * CH : Mh_s;
  ST* ke_s = Ts + CH * KD;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int o = (tid + 512 * j) * (16 / (int)sizeof(ST));
    *reinterpret_cast<V16*>(Mh_s + o) = st_mh[j];
    if constexpr (BF) *reinterpret_cast<V16*>(Ml_s + o) = st_ml[j];
    if constexpr (kStageKe) *reinterpret_cast<V16*>(ke_s + o) = st_ke[j];
  }
  const ST* keA = kStageKe ? ke_s : g_keh;
  if constexpr (!BF) {
    // fp32 mode: M is 64 KB (the 4 loads above covered 32 KB); finish it
#pragma unroll
    for (int j = 4; j < 8; ++j) {
      const int o = (tid + 512 * j) * 4;
      *reinterpret_cast<V16*>(Mh_s + o) = *reinterpret_cast<const V16*>(g_Mh + o);
    }
  }
  __syncthreads();

  // The v rows of this wave's first value tile (16-column tiles, bf16 v) are
  // issued now, ahead of phase 5's loads and stores: they arrive while W, Pn
  // and X are formed.
  constexpr bool kPreV = std::is_same<TV, bf16>::value;
  VRows<TV> vpre;
  if (kPreV && p.Vp < 256 && w < p.Vp / 16) v_rows_issue<TV>(p, b, h, c, 16 * w, l, vpre);

  // ---- phase 5: Pn = -ke^T W ; X = qe - M W  (key tile w; W formed above) ----
  // W^T fragments (rows = key j, k = token), and their negation
  F3 W3[4], W3n[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    float x[8] = {Wc[2 * s][0], Wc[2 * s][1], Wc[2 * s][2], Wc[2 * s][3],
                  Wc[2 * s + 1][0], Wc[2 * s + 1][1], Wc[2 * s + 1][2], Wc[2 * s + 1][3]};
    W3[s] = P::f3(x);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = -x[e];
    W3n[s] = P::f3(x);
  }
  // Pn^T tile (keys 16w.., state rows 16m..): lane (c, q) holds
  // Pn[16m + c][16w + 4q + ii] = element 4(w & 1) + ii of slab w / 2 of Pn's fragment
  const int hofs = 4 * (w & 1);
  auto pn_tile = [&](int m, const F1 (&kb)[4]) {
    f32x4 P0 = zero4();
#pragma unroll
    for (int s = 0; s < 4; ++s) P::m11(P0, P::hi(W3[s]), kb[s]);
    const float x[4] = {-P0[0], -P0[1], -P0[2], -P0[3]};
    SS::st4(g_Pn + fofs(m, w >> 1, l) + hofs, x);
  };
  {
    F1 kb0[4], kb1[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) kb0[s] = SS::fa(keA + fofs(0, s, l));
#pragma unroll 1
    for (int m = 0; m < 8; m += 2) {
#pragma unroll
      for (int s = 0; s < 4; ++s) kb1[s] = SS::fa(keA + fofs(m + 1, s, l));
      pn_tile(m, kb0);
      if (m + 2 < 8) {
#pragma unroll
        for (int s = 0; s < 4; ++s) kb0[s] = SS::fa(keA + fofs(m + 2, s, l));
      }
      pn_tile(m + 1, kb1);
    }
  }
  // X^T tile (keys 16w.., tokens 16rt..): lane (c, q) holds
  // X[16rt + c][16w + 4q + ii] = element 4(w & 1) + ii of slab w / 2 of X's fragment.
  // Operands of tile rt + 1 load while tile rt computes.
  struct XOps {
    f32x4 q0;
    F3 m[4];
  };
  auto ld_x = [&](int rt, XOps& o) {
    o.q0 = *reinterpret_cast<const f32x4*>(g_qe + fofs(rt, w >> 1, l) + hofs);
#pragma unroll
    for (int s = 0; s < 4; ++s)
      if (s <= rt / 2) o.m[s] = SS::fa3(Mh_s + fofs(rt, s, l), Ml_s + fofs(rt, s, l));
  };
  auto x_tile = [&](int rt, const XOps& o) {
    f32x4 X0 = o.q0;
#pragma unroll
    for (int s = 0; s < 4; ++s)
      if (s <= rt / 2) P::m33(X0, W3n[s], o.m[s]);
    const float x[4] = {X0[0], X0[1], X0[2], X0[3]};
    const int xo = fofs(rt, w >> 1, l) + hofs;
    SS::st4s(g_Xh + xo, g_Xl + xo, x);
  };
  {
    XOps xa, xb;
    ld_x(0, xa);
#pragma unroll 1
    for (int rt = 0; rt < 8; rt += 2) {
      ld_x(rt + 1, xb);
      x_tile(rt, xa);
      if (rt + 2 < 8) ld_x(rt + 2, xa);
      x_tile(rt + 1, xb);
    }
  }
  // ---- phase 6: U, Q and (M U)^T of value columns 32g.. (wave w: g = w, w + 8, ..)
  // from the copies of T, M (and in bf16 mode ke^T's high words) phase 5
  // read from LDS; ke^T's low words from the workspace (written in phase 2).
  // One workgroup holding T, ke and M on chip replaces a separate launch
  // that reloaded them once per 32 columns (config 2: 91 vs 94 µs per step,
  // config 5: 3.7 vs 4.2 ms).
  // 32 columns per wave when every wave gets some, else 16 (value heads of 128
  // columns: all 8 waves instead of 4)
  if (p.Vp >= 256) {
    for (int g = w; g < p.Vp / 32; g += 8) {
      VRows<TV> vr;
      v_rows_issue<TV>(p, b, h, c, 32 * g, l, vr);
      value_cols<BF, TV, 2>(p, b, h, c, 32 * g, l, vr, Ts, keA, g_kel, Mh_s, Ml_s);
    }
  } else {
    for (int g = w; g < p.Vp / 16; g += 8) {
      if (!(kPreV && g == w)) v_rows_issue<TV>(p, b, h, c, 16 * g, l, vpre);
      value_cols<BF, TV, 1>(p, b, h, c, 16 * g, l, vpre, Ts, keA, g_kel, Mh_s, Ml_s);
    }
  }
}

// ===========================================================================
// value_cols: U = T (w*v), Q = ke^T U and (M U)^T for value columns
// [col0, col0 + 16 NT) of one chunk unit -- one wave's share, the last phase of
// k_prepass.  The (w*v)^T fragments are formed here from v and w; T, ke^T
// (high / low words) and M (high / low words) are the unit's fragment-native
// arrays (LDS or workspace pointers).
// ===========================================================================
template <bool BF, class TV, int NT>
__device__ __forceinline__ void value_cols(const PF& p, int b, int h, int c, int col0, int l, const VRows<TV>& vr,
                                           const typename Store<BF>::ST* g_T, const typename Store<BF>::ST* g_keh,
                                           const typename Store<BF>::ST* g_kel, const typename Store<BF>::ST* g_Mh,
                                           const typename Store<BF>::ST* g_Ml) {
  using P = Pol<BF>;
  using F1 = typename P::F1;
  using F3 = typename P::F3;
  using SS = Store<BF>;
  using ST = typename SS::ST;
  const int64_t u = ((int64_t)b * p.Hx + h) * p.NCb + c;
  float* g_Q = p.QC + u * (int64_t)(KD * p.Vp);
  float* g_Oi = p.OiT + u * (int64_t)(CH * p.Vp);

  // (w*v)^T fragments of this wave's value columns (rows = column, k = token)
  F3 Bwv[NT][4];
  wv_frags<BF, TV, NT>(p, b, h, c, col0, l, vr, Bwv);
  f32x4 Uc[NT][8];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int rt = 0; rt < 8; ++rt) Uc[nt][rt] = zero4();
#pragma unroll
  for (int rt = 0; rt < 8; ++rt) {
#pragma unroll
    for (int s = 0; s <= rt / 2; ++s) {
      const F1 t = SS::fa(g_T + fofs(rt, s, l));
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) P::m13(Uc[nt][rt], t, Bwv[nt][s]);
    }
    // T read where it is used: keep the scheduler from hoisting every row's
    // fragment reads ahead (that would need them all live at once)
    __builtin_amdgcn_sched_barrier(0);
  }
  // U^T fragments (rows = value column, k = token)
  F3 U3[NT][4];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const float x[8] = {Uc[nt][2 * s][0], Uc[nt][2 * s][1], Uc[nt][2 * s][2], Uc[nt][2 * s][3],
                          Uc[nt][2 * s + 1][0], Uc[nt][2 * s + 1][1], Uc[nt][2 * s + 1][2], Uc[nt][2 * s + 1][3]};
      U3[nt][s] = P::f3(x);
    }
  const int ct0 = col0 / 16;   // value tile of nt = 0 within the execution head
  // Q tiles (rows = key, columns = value), the chain's accumulator layout
  auto q_tile = [&](int m, const F3 (&ka)[4]) {
    f32x4 Qa[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) Qa[nt] = zero4();
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) P::m33(Qa[nt], ka[s], U3[nt][s]);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) *reinterpret_cast<f32x4*>(g_Q + cofs(m, ct0 + nt, p.nct, l)) = Qa[nt];
  };
  auto ld_ke = [&](int m, F3 (&ka)[4]) {
#pragma unroll
    for (int s = 0; s < 4; ++s) ka[s] = SS::fa3(g_keh + fofs(m, s, l), g_kel + fofs(m, s, l));
  };
  {
    F3 kb0[4], kb1[4];
    ld_ke(0, kb0);
#pragma unroll 1
    for (int m = 0; m < 8; m += 2) {
      ld_ke(m + 1, kb1);
      q_tile(m, kb0);
      if (m + 2 < 8) ld_ke(m + 2, kb0);
      q_tile(m + 1, kb1);
    }
  }
  // (M U)^T tiles (rows = value, columns = token), the output kernel's layout
  struct MOps {
    F3 m[4];
  };
  auto ld_m = [&](int rt, MOps& o) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
      if (s <= rt / 2) o.m[s] = SS::fa3(g_Mh + fofs(rt, s, l), g_Ml + fofs(rt, s, l));
  };
  auto oi_tile = [&](int rt, const MOps& o) {
    f32x4 Oa[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) Oa[nt] = zero4();
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (s <= rt / 2) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) P::m33(Oa[nt], U3[nt][s], o.m[s]);
      }
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) *reinterpret_cast<f32x4*>(g_Oi + cofs(rt, ct0 + nt, p.nct, l)) = Oa[nt];
  };
  {
    MOps ma, mb;
    ld_m(0, ma);
#pragma unroll 1
    for (int rt = 0; rt < 8; rt += 2) {
      ld_m(rt + 1, mb);
      oi_tile(rt, ma);
      if (rt + 2 < 8) ld_m(rt + 2, ma);
      oi_tile(rt + 1, mb);
    }
  }
}


// ===========================================================================
// k_chain: S_{c+1} = [same doc] D_c S_c + Pn_c S_c + Q_c, and the output
// O_c = X_c S_c + Oi_c of every chunk, for one 16-column value tile of one
// exec head.  One workgroup of 8 waves in two roles that meet at one LDS
// barrier per chunk:
//   waves 0-3 (recurrence): wave w owns state rows 32w..32w+31 (fp32, in
//     VGPRs) and publishes them to LDS as slab w of the S_c^T fragment
//     (split high / low bf16 in bf16 mode); after the barrier it reads the
//     whole fragment and forms S_{c+1}: two independent chains of 4 MFMAs
//     on the sequential path.
//   waves 4-7 (output): wave 4 + t computes token tiles 2t and 2t + 1 of the
//     chunk as O^T = S^T X^T + (M U)^T from the same fragments, beside the
//     recurrence on the other wave slot of each SIMD.
// A chunk step is short next to the latency of its operand loads, so each
// role keeps several chunks of operands in flight in VGPRs (ChainSets: the
// number of operand sets; a chunk's loads are issued that many steps minus
// one ahead).  Two waves per SIMD leave each wave 256 VGPRs for them.
// The role is a scalar (wave-uniform) branch, and both roles execute exactly
// one barrier per chunk.  Loop trips run whole groups of chunks and the
// remainder runs after the loop: an exit in the middle of a trip would make
// the loop head wait for every outstanding load, the prefetches included.
// ===========================================================================
// (one tile: 2 and 3 sets, config 2 chain 28.4-28.8 to 27.8 us and config 5
// 1325-1336 to 1300-1304 us against 4 and 3; several tiles per workgroup: one
// recurrence set, the registers two would hold spilled, config 3 chain
// 492-502 to 434-438 us)
template <bool BF, int NTL> struct ChainSets {
  static constexpr int rec = NTL == 1 ? 2 : 1, out = NTL == 1 ? 3 : 2;
};
template <int NTL> struct ChainSets<false, NTL> {   // fp32 fragments are twice as wide
  static constexpr int rec = 2, out = 3;
};

// NTL: 16-column tiles per workgroup.  One tile per workgroup spreads a
// head's columns over the most CUs (config 2: 192 workgroups); when the tiles
// outnumber the CUs, a workgroup takes NTL tiles of one value head, so each
// chunk's Pn and X fragments are loaded once for all of them (the CU's load
// rate bounds a step: one tile loads 112 KB per chunk, NTL tiles 48 + 64 NTL).
template <bool BF, class TO, int NTL>
__global__ __launch_bounds__(512) void k_chain(const PF p) {
  using P = Pol<BF>;
  using F1 = typename P::F1;
  using F3 = typename P::F3;
  using SS = Store<BF>;
  using ST = typename SS::ST;
  constexpr int NT = 512;
  constexpr int FR = 4 * 64 * 8;   // elements of one tile's S^T fragment
  // S_c^T fragments of the NTL tiles, high and low words, double-buffered
  __shared__ __align__(16) ST Sh_s[2][NTL][FR];
  __shared__ __align__(16) ST Sl_s[2][NTL][BF ? FR : 1];
  __shared__ int flg[2 * kMaxBlockChunks];   // is_new_doc, all_same_doc per chunk
  const int tid = threadIdx.x;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l = tid & 63, r16 = l & 15, q = l >> 4;
  int ctg, h, b;
  xcd_block(ctg, h, b);
  const int ct0 = NTL * ctg;       // first tile; the NTL tiles lie in one value head
  const int hv = p.gates_at_hv ? h : h * p.G + (16 * ct0) / KD;
  const int vc0 = (16 * ct0) % KD;   // first column of the tiles inside head hv
  auto frag_lo = [&](int buf, int j) -> ST* { return BF ? &Sl_s[buf][j][0] : &Sh_s[buf][j][0]; };
  // chunk flags into LDS once, so testing them never waits on vector loads
  for (int i = tid; i < 2 * p.NCb; i += NT) flg[i] = p.flags[(int64_t)b * p.NCb * 2 + i];
  __syncthreads();

  if (wid < 4) {
    // ---------------- recurrence: state rows 32w.. ----------------
    constexpr int RS = ChainSets<BF, NTL>::rec;
    const int w = wid;
    const int64_t sbase = ((int64_t)b * p.Hv + hv) * KD * KD + vc0 + r16;
    f32x4 S[NTL][2];
#pragma unroll
    for (int j = 0; j < NTL; ++j)
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int ii = 0; ii < 4; ++ii)
          S[j][r][ii] = p.has_init ? p.init[sbase + 16 * j + (int64_t)(32 * w + 16 * r + 4 * q + ii) * KD] : 0.f;
    struct Ops {
      F1 pf[2][4];
      f32x4 qc[NTL][2], dv[2];
    };
    auto load_ops = [&](int c, Ops& o) {
      const int cc = min(c, p.NCb - 1);
      const int64_t u = ((int64_t)b * p.Hx + h) * p.NCb + cc;
      const ST* Pn = (const ST*)p.PnA + u * (KD * KD);
      const float* Qc = p.QC + u * (int64_t)(KD * p.Vp);
#pragma unroll
      for (int r = 0; r < 2; ++r) {
#pragma unroll
        for (int s = 0; s < 4; ++s) o.pf[r][s] = SS::fa(Pn + fofs(2 * w + r, s, l));
#pragma unroll
        for (int j = 0; j < NTL; ++j) o.qc[j][r] = *reinterpret_cast<const f32x4*>(Qc + cofs(2 * w + r, ct0 + j, p.nct, l));
        o.dv[r] = *reinterpret_cast<const f32x4*>(p.dvec + u * KD + 32 * w + 16 * r + 4 * q);
      }
    };
    auto step = [&](int c, const Ops& o) {
      const int is_new = flg[2 * c], same = flg[2 * c + 1];
      const int fo = (w * 64 + l) * 8;
#pragma unroll
      for (int j = 0; j < NTL; ++j) {
        if (is_new) { S[j][0] = zero4(); S[j][1] = zero4(); }
        // lane (n, q) holds rows 32w + 16r + 4q + ii = element 4r + ii of slab w
        const float x[8] = {S[j][0][0], S[j][0][1], S[j][0][2], S[j][0][3],
                            S[j][1][0], S[j][1][1], S[j][1][2], S[j][1][3]};
        SS::st8s(&Sh_s[c & 1][j][fo], frag_lo(c & 1, j) + fo, x);
      }
      lds_barrier();
#pragma unroll
      for (int j = 0; j < NTL; ++j) {
        F1 Sf[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) Sf[s] = SS::fa(&Sh_s[c & 1][j][(s * 64 + l) * 8]);
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          f32x4 acc = o.qc[j][r];
#pragma unroll
          for (int s = 0; s < 4; ++s) P::m11(acc, o.pf[r][s], Sf[s]);
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) S[j][r][ii] = acc[ii] + (same ? o.dv[r][ii] * S[j][r][ii] : 0.f);
        }
      }
    };
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
    const int rem = p.NCb - RS * ntrip;   // < RS; their operands are loaded
#pragma unroll
    for (int jj = 0; jj + 1 < RS; ++jj)
      if (jj < rem) step(RS * ntrip + jj, o[jj]);
#pragma unroll
    for (int j = 0; j < NTL; ++j)
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) p.fin[sbase + 16 * j + (int64_t)(32 * w + 16 * r + 4 * q + ii) * KD] = S[j][r][ii];
  } else {
    // ---------------- output: token tiles 2t, 2t + 1 ----------------
    constexpr int OS = ChainSets<BF, NTL>::out;
    const int t2 = 2 * (wid - 4);
    struct Ops {
      F3 xb[2][4];        // X fragments of the two token tiles (all NTL column tiles use them)
      f32x4 oi[NTL][2];   // (M U)^T tiles of the two token tiles
    };
    auto load_ops = [&](int c, Ops& o) {
      const int cc = min(c, p.NCb - 1);
      const int64_t u = ((int64_t)b * p.Hx + h) * p.NCb + cc;
      const ST* Xh = (const ST*)p.XAh + u * (CH * KD);
      const ST* Xl = (const ST*)p.XAl + u * (CH * KD);
#pragma unroll
      for (int r = 0; r < 2; ++r) {
#pragma unroll
        for (int s = 0; s < 4; ++s) o.xb[r][s] = SS::fa3(Xh + fofs(t2 + r, s, l), Xl + fofs(t2 + r, s, l));
#pragma unroll
        for (int j = 0; j < NTL; ++j)
          o.oi[j][r] = *reinterpret_cast<const f32x4*>(p.OiT + u * (int64_t)(CH * p.Vp) + cofs(t2 + r, ct0 + j, p.nct, l));
      }
    };
    f32x4 res[NTL][2];
    auto step = [&](int c, const Ops& o) {
      lds_barrier();
#pragma unroll
      for (int j = 0; j < NTL; ++j) {
        res[j][0] = o.oi[j][0];
        res[j][1] = o.oi[j][1];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int fs = (s * 64 + l) * 8;
          const F3 sf = SS::fa3(&Sh_s[c & 1][j][fs], frag_lo(c & 1, j) + fs);
          P::m33(res[j][0], sf, o.xb[0][s]);
          P::m33(res[j][1], sf, o.xb[1][s]);
        }
      }
    };
    // lane (t, q) holds O[token 16 (t2 + r) + t][column 16 (ct0 + j) + 4q + ii].
    // Every lane stores (tokens past the end into the workspace's sink): a
    // store skipped under a branch would leave the compiler unsure how many
    // vector-memory operations are pending at the loop head, and it would
    // then wait for all of them (the prefetches included).
    auto store = [&](int c) {
#pragma unroll
      for (int j = 0; j < NTL; ++j) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const int t = p.t0 + c * CH + 16 * (t2 + r) + r16;
          const bool tv = t < min(p.t0 + p.nt, p.L);
          const int64_t ob = (((int64_t)b * p.L + (tv ? t : 0)) * p.Hv + hv) * KD + vc0 + 16 * j + 4 * q;
          TO* dst = tv ? (TO*)p.out + ob : (TO*)p.sink + 4 * l;
          const float x[4] = {res[j][r][0], res[j][r][1], res[j][r][2], res[j][r][3]};
          st4<TO>(dst, x);
        }
      }
    };
    // Each chunk's prefetch is issued before its output store: the wait for
    // a prefetched operand then never covers a store (the vector-memory
    // counter counts stores too and drains in order).
    Ops o[OS];
#pragma unroll
    for (int jj = 0; jj + 1 < OS; ++jj) load_ops(jj, o[jj]);
    const int ntrip = p.NCb / OS;
#pragma unroll 1
    for (int k = 0; k < ntrip; ++k) {
#pragma unroll
      for (int jj = 0; jj < OS; ++jj) {
        step(OS * k + jj, o[jj]);
        load_ops(OS * k + jj + OS - 1, o[(jj + OS - 1) % OS]);
        store(OS * k + jj);
      }
    }
    const int rem = p.NCb - OS * ntrip;
#pragma unroll
    for (int jj = 0; jj + 1 < OS; ++jj)
      if (jj < rem) {
        step(OS * ntrip + jj, o[jj]);
        store(OS * ntrip + jj);
      }
  }
}

// ===========================================================================
// host side
// ===========================================================================
namespace {

struct WsLayout {
  size_t flags, dvec, PnA, QC, XAh, XAl, OiT, BeB, KeBh, KeBl, MAh, MAl, QeA, sink, carry, total;
};

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Split operands (X, St, ke^T, M) have a low-word array in bf16 mode only.
WsLayout ws_layout(const dn_prefill_args* a, int Hx, int Vp, int NCb, bool bf) {
  WsLayout L{};
  const size_t es = bf ? 2 : 4;
  const size_t ls = bf ? 2 : 0;
  const size_t units = (size_t)a->B * Hx * NCb;
  const size_t sq = (size_t)CH * KD;   // elements of one 128 x 128 operand
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off += align256(bytes); return o; };
  L.flags = take((size_t)a->B * NCb * 2 * 4);
  L.dvec = take(units * KD * 4);
  L.PnA = take(units * sq * es);
  L.QC = take(units * KD * Vp * 4);
  L.XAh = take(units * sq * es);
  L.XAl = take(units * sq * ls);
  L.OiT = take(units * CH * Vp * 4);
  L.BeB = take(units * sq * es);
  L.KeBh = take(units * sq * es);
  L.KeBl = take(units * sq * ls);
  L.MAh = take(units * sq * es);
  L.MAl = take(units * sq * ls);
  L.QeA = take(units * sq * 4);
  L.sink = take(64 * 16);
  L.carry = take((size_t)a->B * a->Hv * KD * KD * 4);
  L.total = off;
  return L;
}

// Workspace budget of one call (token blocks beyond it run one after another).
// Larger blocks mean fewer launches and longer chains per launch: at BASELINE
// config 3 (8192 units) a 4 GiB budget measured 2.64 ms per call against
// 2.91 ms at 160 MiB, and config 5's 8192-token streaming blocks run in one
// launch each (4.15 ms against 5.47 ms); config 2 (147 MB) is unaffected.
constexpr size_t kAutoBudget = size_t(4096) << 20;

// Chunks per token block: block_tokens when given, else the most that keep
// the workspace within kAutoBudget.  A hard budget (the allocation-free entry
// point's scratch) also caps a given block_tokens.
int block_chunks(const dn_prefill_args* a, int Hx, int Vp, size_t budget = 0) {
  const int nct = (a->nt + CH - 1) / CH;
  int ncb = std::min(nct, kMaxBlockChunks);
  if (a->block_tokens > 0) {
    ncb = std::max(1, std::min(ncb, a->block_tokens / CH));
    if (budget == 0) return ncb;
  }
  if (budget == 0) budget = kAutoBudget;
  const bool bf = a->precision == 0;
  while (ncb > 1 && ws_layout(a, Hx, Vp, ncb, bf).total > budget) ncb = (ncb + 1) / 2;
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

int g_chain_tiles = -1;   // -1: unread; 0: by grid size; 1, 2, 4: forced (DN_CHAIN_TILES, measurements)
int chain_tiles() {
  if (g_chain_tiles < 0) {
    const char* e = getenv("DN_CHAIN_TILES");
    const int v = e ? atoi(e) : 0;
    g_chain_tiles = (v == 1 || v == 2 || v == 4) ? v : 0;
  }
  return g_chain_tiles;
}

int g_prepass_scalar = -1;   // -1: unread; 0: general path forced (DN_PREPASS_SCALAR=0, measurements)

// One decay and one b per (token, head) with bf16 q / k in precision "bf16"
// (the Gated DeltaNet form) runs the scalar-gate prepass.
bool scalar_gates(const PF& p) {
  if (g_prepass_scalar < 0) {
    const char* e = getenv("DN_PREPASS_SCALAR");
    g_prepass_scalar = (e && atoi(e) == 0) ? 0 : 1;
  }
  return g_prepass_scalar == 1 && p.g_c == 1 && p.b_c == 1 && !p.fuse;
}

template <bool BF, class TIn, class TV>
hipError_t launch_all(const PF& p, hipStream_t st) {
  prof_mark(0, st, false);
  bool sc = false;
  if constexpr (BF && std::is_same<TIn, bf16>::value) {
    sc = scalar_gates(p);
    if (sc) hipLaunchKernelGGL((k_prepass<BF, TIn, TV, true>), dim3(p.B * p.Hx * p.NCb), dim3(512), 0, st, p);
  }
  if (!sc) hipLaunchKernelGGL((k_prepass<BF, TIn, TV, false>), dim3(p.B * p.Hx * p.NCb), dim3(512), 0, st, p);
  prof_mark(0, st, true);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  prof_mark(2, st, false);
  // several column tiles per workgroup once the tiles outnumber the CUs
  // (bf16 mode; config 3: 1024 tiles)
  const int tiles = (p.Vp / 16) * p.Hx * p.B;
  int ntl = 1;
  if constexpr (BF) {
    ntl = chain_tiles();
    if (ntl == 0) ntl = tiles >= 4 * 256 ? 4 : (tiles >= 2 * 256 ? 2 : 1);
    if (ntl == 4)
      hipLaunchKernelGGL((k_chain<BF, TV, 4>), dim3(p.Vp / 64, p.Hx, p.B), dim3(512), 0, st, p);
    else if (ntl == 2)
      hipLaunchKernelGGL((k_chain<BF, TV, 2>), dim3(p.Vp / 32, p.Hx, p.B), dim3(512), 0, st, p);
  }
  if (ntl == 1) hipLaunchKernelGGL((k_chain<BF, TV, 1>), dim3(p.Vp / 16, p.Hx, p.B), dim3(512), 0, st, p);
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

namespace {

// One dn_prefill_fwd call in token blocks of ncb chunks over the workspace ws.
int prefill_run(const dn_prefill_args* a, char* ws, size_t workspace_bytes, int ncb, hipStream_t st) {
  const int G = a->Hv / a->Hk;
  const int Hx = a->gates_at_hv ? a->Hv : a->Hk;
  const int Vp = a->gates_at_hv ? KD : G * KD;
  const bool bf = a->precision == 0;
  const WsLayout Lw = ws_layout(a, Hx, Vp, ncb, bf);
  if (ws == nullptr || workspace_bytes < Lw.total) return set_error(DN_E_WORKSPACE, "workspace too small");

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
  p.flags = (int32_t*)(ws + Lw.flags);
  p.dvec = (float*)(ws + Lw.dvec);
  p.nct = Vp / 16;
  p.PnA = ws + Lw.PnA;
  p.QC = (float*)(ws + Lw.QC);
  p.XAh = ws + Lw.XAh;
  p.XAl = bf ? ws + Lw.XAl : p.XAh;
  p.OiT = (float*)(ws + Lw.OiT);
  p.BeB = ws + Lw.BeB;
  p.KeBh = ws + Lw.KeBh;
  p.KeBl = bf ? ws + Lw.KeBl : p.KeBh;
  p.MAh = ws + Lw.MAh;
  p.MAl = bf ? ws + Lw.MAl : p.MAh;
  p.QeA = (float*)(ws + Lw.QeA);
  p.sink = ws + Lw.sink;
  float* carry = a->final_state ? a->final_state : (float*)(ws + Lw.carry);

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

int prefill_shape_ok(const dn_prefill_args* a) {
  const int rc = check_args(a);
  if (rc != DN_OK) return rc;
  const int G = a->Hv / a->Hk;
  const int Vp = a->gates_at_hv ? KD : G * KD;
  if (Vp % 64 != 0 || Vp > 1024) return set_error(DN_E_INVALID, "value width per execution head must be 64..1024");
  return DN_OK;
}

}  // namespace

extern "C" int dn_prefill_fwd(const dn_prefill_args* a, void* workspace, size_t workspace_bytes, void* stream) {
  const int rc = prefill_shape_ok(a);
  if (rc != DN_OK) return rc;
  const int Hx = a->gates_at_hv ? a->Hv : a->Hk;
  const int Vp = a->gates_at_hv ? KD : (a->Hv / a->Hk) * KD;
  return prefill_run(a, (char*)workspace, workspace_bytes, block_chunks(a, Hx, Vp), (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
// Allocation-free prefill: dn_prefill_fwd over a file-scope device scratch
// array instead of a caller workspace.  Each GPU holds its own copy of
// `scratch` (DN_NOALLOC_SCRATCH_BYTES) from the library's first use on it
// until the process ends.  Host code never passes the array's name to a
// kernel (on the host it is only a stand-in for the symbol): the device
// address comes from hipGetSymbolAddress, taken once per device with that
// device current, and is the only handle used afterwards.
// ---------------------------------------------------------------------------
namespace {

static __device__ __align__(256) char scratch[DN_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
char* g_scratch_ptr[kMaxDevices] = {};

// the current device's address of `scratch` (nullptr and an error set on failure)
char* scratch_address() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error(DN_E_LAUNCH, "no current HIP device");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      set_error(DN_E_LAUNCH, e != hipSuccess ? hipGetErrorString(e) : "null scratch address");
      return nullptr;
    }
    g_scratch_ptr[dev] = (char*)ptr;
  }
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" int dn_prefill_fwd_noalloc(const dn_prefill_args* a, void* stream) {
  const int rc = prefill_shape_ok(a);
  if (rc != DN_OK) return rc;
  const int Hx = a->gates_at_hv ? a->Hv : a->Hk;
  const int Vp = a->gates_at_hv ? KD : (a->Hv / a->Hk) * KD;
  const int ncb = block_chunks(a, Hx, Vp, DN_NOALLOC_SCRATCH_BYTES);
  if (ws_layout(a, Hx, Vp, ncb, a->precision == 0).total > DN_NOALLOC_SCRATCH_BYTES)
    return set_error(DN_E_WORKSPACE,
                     "dn_prefill_fwd_noalloc: one 128-token chunk of every (batch, head) needs more than "
                     "DN_NOALLOC_SCRATCH_BYTES of scratch; use dn_prefill_fwd with a workspace");
  char* ws = scratch_address();
  if (ws == nullptr) return DN_E_LAUNCH;
  return prefill_run(a, ws, DN_NOALLOC_SCRATCH_BYTES, ncb, (hipStream_t)stream);
}
