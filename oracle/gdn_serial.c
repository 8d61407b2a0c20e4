/*
 * Token-serial GDN-2 recurrence in plain C -- TEST INFRASTRUCTURE ONLY.
 *
 * Used by tests/ (cross-check of the NumPy oracle, and large-shape head
 * subsets) and by the cpu_baseline leg of bench.py (timed as the "port"
 * CPU baseline).  The product library never links or calls it.
 *
 * Restates the per-token recurrence of the reference's token_serial_gdn2
 * (maelie-labs/deltanet-tpu, src/deltanet_tpu/reference.py:123-161):
 *
 *   reset S when seg[t] != seg[t-1]                    (reference.py:127-129)
 *   S  <- diag(exp(g_t)) S                             (reference.py:131-133)
 *   e   = S^T (b_t * k_t);  vn = w_t * v_t - e          (reference.py:135-140)
 *   S  <- S + k_t vn^T;     o_t = S^T q_t               (reference.py:142-146)
 *
 * Inputs are already prepared by the caller (normalised / scaled q and k,
 * activated and clamped gates, canonical segment ids).  Gates carry their own
 * head count Hx in {1, Hk, Hv} (value head hv reads head hv // (Hv/Hx), or 0)
 * and channel count Cx in {1, K or V} (stride 0 when 1).
 *
 * Parallelism: OpenMP over (batch, value head) chains when built with
 * -fopenmp; the inner loops are written so gcc -O3 vectorises them.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define DEFINE_SERIAL(T, NAME)                                                                 \
  int NAME(int B, int L, int Hk, int Hv, int K, int V, const T* q, const T* k, const T* v,     \
           const T* g, int Hg, int Cg, const T* b, int Hb, int Cb, const T* w, int Hw, int Cw, \
           const int64_t* seg, const T* init_state, const int64_t* prev_seg, T* out,          \
           T* final_state, int nthreads) {                                                     \
    if (B <= 0 || L < 0 || Hk <= 0 || Hv <= 0 || Hv % Hk) return -1;                          \
    const int G = Hv / Hk;                                                                     \
    const int nchain = B * Hv;                                                                 \
    int err = 0;                                                                               \
    (void)nthreads;                                                                            \
    _Pragma("omp parallel for schedule(dynamic, 1) num_threads(nthreads) reduction(|:err)")    \
    for (int ch = 0; ch < nchain; ++ch) {                                                      \
      const int bb = ch / Hv, hv = ch % Hv, hk = hv / G;                                       \
      const int hg = (Hg == 1) ? 0 : hv / (Hv / Hg);                                           \
      const int hb = (Hb == 1) ? 0 : hv / (Hv / Hb);                                           \
      const int hw = (Hw == 1) ? 0 : hv / (Hv / Hw);                                           \
      T* S = (T*)malloc(sizeof(T) * (size_t)K * V);                                            \
      T* e = (T*)malloc(sizeof(T) * (size_t)V);                                                \
      T* d = (T*)malloc(sizeof(T) * (size_t)K);                                                \
      if (!S || !e || !d) { err |= 1; free(S); free(e); free(d); continue; }                    \
      if (init_state)                                                                          \
        memcpy(S, init_state + ((size_t)bb * Hv + hv) * K * V, sizeof(T) * (size_t)K * V);     \
      else                                                                                     \
        memset(S, 0, sizeof(T) * (size_t)K * V);                                               \
      int64_t prev = prev_seg ? prev_seg[bb] : (init_state ? seg[(size_t)bb * L] : -1);         \
      for (int t = 0; t < L; ++t) {                                                            \
        const size_t bt = (size_t)bb * L + t;                                                  \
        const int64_t st = seg[bt];                                                            \
        if (st != prev) memset(S, 0, sizeof(T) * (size_t)K * V);                               \
        prev = st;                                                                             \
        const T* qt = q + (bt * Hk + hk) * K;                                                  \
        const T* kt = k + (bt * Hk + hk) * K;                                                  \
        const T* vt = v + (bt * Hv + hv) * V;                                                  \
        const T* gt = g + (bt * Hg + hg) * Cg;                                                 \
        const T* btp = b + (bt * Hb + hb) * Cb;                                                \
        const T* wt = w + (bt * Hw + hw) * Cw;                                                 \
        for (int i = 0; i < K; ++i) d[i] = (T)exp(gt[Cg == 1 ? 0 : i]);                        \
        for (int j = 0; j < V; ++j) e[j] = 0;                                                  \
        for (int i = 0; i < K; ++i) {                                                          \
          const T di = d[i];                                                                   \
          const T bi = btp[Cb == 1 ? 0 : i] * kt[i];                                           \
          T* Si = S + (size_t)i * V;                                                           \
          for (int j = 0; j < V; ++j) {                                                        \
            Si[j] *= di;                                                                       \
            e[j] += bi * Si[j];                                                                \
          }                                                                                    \
        }                                                                                      \
        for (int j = 0; j < V; ++j) e[j] = wt[Cw == 1 ? 0 : j] * vt[j] - e[j];                 \
        T* ot = out + (bt * Hv + hv) * V;                                                      \
        for (int j = 0; j < V; ++j) ot[j] = 0;                                                 \
        for (int i = 0; i < K; ++i) {                                                          \
          const T ki = kt[i], qi = qt[i];                                                      \
          T* Si = S + (size_t)i * V;                                                           \
          for (int j = 0; j < V; ++j) {                                                        \
            Si[j] += ki * e[j];                                                                \
            ot[j] += qi * Si[j];                                                               \
          }                                                                                    \
        }                                                                                      \
      }                                                                                        \
      if (final_state)                                                                         \
        memcpy(final_state + ((size_t)bb * Hv + hv) * K * V, S, sizeof(T) * (size_t)K * V);    \
      free(S);                                                                                 \
      free(e);                                                                                 \
      free(d);                                                                                 \
    }                                                                                          \
    return err ? -2 : 0;                                                                       \
  }

DEFINE_SERIAL(double, dn_oracle_serial_f64)
DEFINE_SERIAL(float, dn_oracle_serial_f32)
