// Single-token GDN-2 decode step on gfx950: a pure HBM stream of the
// (B, Hv, K, V) state.  One workgroup of 256 lanes owns one (batch, value
// head) 128x128 state: it reads the state once with 16-byte non-temporal
// loads, keeps it in VGPRs, and writes the updated state once.
//
// Reference: gdn2_decode_step (maelie-labs/deltanet-tpu v0.3.0,
// src/deltanet_tpu/gdn2.py:2289-2490):
//   g <- min(g, 0) (+ guard clamps)                 gdn2.py:2393-2402
//   S <- 0 where reset                              gdn2.py:2404-2412
//   q, k repeated to value heads (hv // G)          gdn2.py:2414-2448
//   q <- scale q / sqrt(|q|^2 + 1e-6) (if l2norm)   gdn2.py:2434-2438
//   Sd = e^g (rows) * S ; e = Sd^T (b k) ; vn = w v - e
//   S' = Sd + k vn^T ; o = S'^T q                   gdn2.py:2471-2478
//   cap |S'|_F at tau (guard), cast to state dtype  gdn2.py:2484-2489
// The read-out uses o_j = sum_i q_i d_i S_ij + (q.k) vn_j, which equals
// S'^T q exactly in real arithmetic and needs only the single pass over S.
#include <atomic>
#include <mutex>
#include <string>
#include <vector>

#include "dn_common.h"
#include "dn_host.h"

namespace dn {

namespace {
thread_local std::string g_last_error;
}

int set_error(int code, const char* msg) {
  g_last_error = msg ? msg : "";
  return code;
}

namespace {
// Profiling records are process-wide (a framework may launch the backward from
// its own thread); the event opened by a launch's first mark is per thread.
struct ProfRec { int kind; hipEvent_t a, b; };
std::atomic<bool> g_prof{false};
std::mutex g_prof_mu;
std::vector<ProfRec> g_recs;
std::vector<hipEvent_t> g_pool;
thread_local hipEvent_t g_open = nullptr;

hipEvent_t take_event() {
  {
    std::lock_guard<std::mutex> lk(g_prof_mu);
    if (!g_pool.empty()) { hipEvent_t e = g_pool.back(); g_pool.pop_back(); return e; }
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}
}  // namespace

bool profiling() { return g_prof.load(); }

void prof_mark(int kind, hipStream_t st, bool after) {
  if (!g_prof.load()) return;
  hipEvent_t e = take_event();
  if (e == nullptr) return;
  (void)hipEventRecord(e, st);
  if (!after) {
    g_open = e;
  } else if (g_open != nullptr) {
    std::lock_guard<std::mutex> lk(g_prof_mu);
    g_recs.push_back(ProfRec{kind, g_open, e});
    g_open = nullptr;
  }
}

struct DP {
  int B, Hk, Hv, G;
  const void *q, *k, *v;
  int qk_dt, v_dt;
  const void* g; int g_dt, g_h, g_c;
  const void* b; int b_dt, b_h, b_c;
  const void* w; int w_dt, w_h, w_c;
  const void* sin;
  void* sout;
  const uint8_t* reset;
  void* out;
  float scale; int l2norm, guard; float tau;
  int T;   // tokens per call (dn_decode_steps); per-token tensors carry a T axis after B
};

__device__ __forceinline__ int dgate_head(int H, int Hk, int Hv, int hv, int G) {
  if (H == 1) return 0;
  return (H == Hv) ? hv : hv / G;
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

// State loads and stores are non-temporal: each byte is touched once per
// step, so it should not displace cached lines (measured faster than plain
// loads and stores at config 4).
template <class T> __device__ __forceinline__ T ldg(const T* p) { return __builtin_nontemporal_load(p); }
template <class T> __device__ __forceinline__ void stg(T* p, const T& x) { __builtin_nontemporal_store(x, p); }

// 8 state elements of one row held by one lane, kept in the stored format
// until use: 8 consecutive bf16 (one 16-byte load), or for fp32 columns
// 4c..4c+3 and 64+4c..64+4c+3 (two 16-byte loads that each cover 256
// contiguous bytes of the row across the 16 column lanes).
template <class T> struct Row8;
template <> struct Row8<bf16> {
  bf16x8 a;
  __device__ __forceinline__ void load(const bf16* row, int cg) { a = ldg(reinterpret_cast<const bf16x8*>(row + 8 * cg)); }
  __device__ __forceinline__ void zero() { a = bf16x8{}; }
  __device__ __forceinline__ float at(int e) const { return (float)a[e]; }
  // the same value through an opaque instruction: the compiler cannot reuse
  // an earlier conversion, so it keeps the 4 packed words live instead of 8
  // expanded floats between the two passes over the state
  __device__ __forceinline__ float at2(int e) const {
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    const uint32_t wd = __builtin_bit_cast(u4, a)[e >> 1];
    uint32_t r;
    if (e & 1) asm("v_and_b32 %0, 0xffff0000, %1" : "=v"(r) : "v"(wd));
    else asm("v_lshlrev_b32 %0, 16, %1" : "=v"(r) : "v"(wd));
    return __builtin_bit_cast(float, r);
  }
  static __device__ __forceinline__ int col(int cg, int e) { return 8 * cg + e; }
  static __device__ __forceinline__ void store(bf16* row, int cg, const float* y) {
    bf16x8 h;
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = (bf16)y[e];
    stg(reinterpret_cast<bf16x8*>(row + 8 * cg), h);
  }
};
template <> struct Row8<float> {
  f32x4 a, b;
  __device__ __forceinline__ void load(const float* row, int cg) {
    a = ldg(reinterpret_cast<const f32x4*>(row + 4 * cg));
    b = ldg(reinterpret_cast<const f32x4*>(row + 64 + 4 * cg));
  }
  __device__ __forceinline__ void zero() { a = zero4(); b = zero4(); }
  __device__ __forceinline__ float at(int e) const { return e < 4 ? a[e] : b[e - 4]; }
  __device__ __forceinline__ float at2(int e) const { return at(e); }
  static __device__ __forceinline__ int col(int cg, int e) { return e < 4 ? 4 * cg + e : 60 + 4 * cg + e; }
  static __device__ __forceinline__ void store(float* row, int cg, const float* y) {
    stg(reinterpret_cast<f32x4*>(row + 4 * cg), f32x4{y[0], y[1], y[2], y[3]});
    stg(reinterpret_cast<f32x4*>(row + 64 + 4 * cg), f32x4{y[4], y[5], y[6], y[7]});
  }
};
// writes the 8 values of one lane's row segment in the output state format,
// at the columns the input format gave that lane
template <class TSin, class TSout>
__device__ __forceinline__ void store_row(TSout* row, int cg, const float* y) {
  if constexpr (sizeof(TSin) == sizeof(TSout)) {
    Row8<TSin>::store(row, cg, y);
  } else if constexpr (sizeof(TSin) == 4) {           // fp32 in, bf16 out
    bf16x4 lo, hi;
#pragma unroll
    for (int e = 0; e < 4; ++e) { lo[e] = (bf16)y[e]; hi[e] = (bf16)y[4 + e]; }
    stg(reinterpret_cast<bf16x4*>(row + 4 * cg), lo);
    stg(reinterpret_cast<bf16x4*>(row + 64 + 4 * cg), hi);
  } else {                                            // bf16 in, fp32 out
    stg(reinterpret_cast<f32x4*>(row + 8 * cg), f32x4{y[0], y[1], y[2], y[3]});
    stg(reinterpret_cast<f32x4*>(row + 8 * cg + 4), f32x4{y[4], y[5], y[6], y[7]});
  }
}

// waves per workgroup of the single-step kernel: 2 (16 state rows per lane)
// measured 3% faster than 4 and 10% faster than 8 at config 4 (bf16 state)
constexpr int kDecodeWaves = 2;
constexpr int kMultiWaves = 4;   // waves per workgroup of the T-token kernel (8 measured slower)

// One workgroup of NW waves per (batch row, value head).  Lane (rg, cg)
// holds R = 32/NW state rows, 8 columns per row (Row8 above): for a bf16
// state rows rg + 4*NW*r, so the 4 row groups of a wave read 4 consecutive
// rows (1 KB contiguous) per load instruction (consecutive rows per lane
// measured 4% slower at config 4); for an fp32 state rows R*rg + r (the
// interleaved order measured 0.5% slower there).  Every global load is
// issued at entry so their latencies overlap: q, k, gates and v first, then
// the state, so the normalisation and its barriers (which wait only for the
// first ones) run while the state is still arriving (fp32 182 to 177 us,
// bf16 94.0 to 93.3 us at config 4).  The state loads and stores are
// non-temporal (each byte is touched once per step).  The column sums reduce inside each wave by
// shuffles, then across the NW waves through LDS.
template <class TSin, class TSout, int NW, int HPW>
__global__ __launch_bounds__(64 * NW * HPW) void k_decode(const DP p) {
  constexpr int K = 128, V = 128, R = K / (4 * NW);   // rows per lane
  static_assert(NW >= 2 && K % (4 * NW) == 0, "waves per workgroup");
  using RowIn = Row8<TSin>;
  __shared__ float qn_[HPW][K], kn_[HPW][K], dd_[HPW][K], bt_[HPW][K], vn_[HPW][V];
  __shared__ float red_[HPW][2][NW][V];
  __shared__ float rbuf_[HPW][3][2];
  __shared__ float gbuf_[HPW][NW];
  // HPW (batch row, value head) matrices per workgroup, NW waves each; the
  // barriers are shared
  const int hs = HPW == 1 ? 0 : (int)threadIdx.x / (64 * NW);
  float* qn = qn_[hs]; float* kn = kn_[hs]; float* dd = dd_[hs]; float* bt = bt_[hs]; float* vn = vn_[hs];
  auto& red = red_[hs];
  auto& rbuf = rbuf_[hs];
  auto& gbuf = gbuf_[hs];

  const int tid = HPW == 1 ? (int)threadIdx.x : (int)threadIdx.x & (64 * NW - 1);
  const int lane = tid & 63, wid = tid >> 6;
  const int cg = tid & 15, rg = tid >> 4;
  const int bh_raw = blockIdx.x * HPW + hs;
  const bool valid = HPW == 1 || bh_raw < p.B * p.Hv;   // an odd count leaves the last half idle
  const int bh = valid ? bh_raw : p.B * p.Hv - 1;
  const int bb = bh / p.Hv, hv = bh % p.Hv;
  const int hk = hv / p.G;
  const bool rst = p.reset != nullptr && p.reset[bb] != 0;
  const int64_t sbase = (int64_t)bh * K * V;

  // lanes 0-127: element i = tid of q, k, g, b and column j = tid of w, v
  const int i = tid;
  float xq = 0.f, xk = 0.f, gv = 0.f, bv = 0.f, wv = 0.f, vv = 0.f;
  if (tid < 128) {
    const int64_t qo = ((int64_t)bb * p.Hk + hk) * K + i;
    xq = ld_f(p.q, qo, p.qk_dt);
    xk = ld_f(p.k, qo, p.qk_dt);
    const int hg = dgate_head(p.g_h, p.Hk, p.Hv, hv, p.G);
    const int hb = dgate_head(p.b_h, p.Hk, p.Hv, hv, p.G);
    const int hw = dgate_head(p.w_h, p.Hk, p.Hv, hv, p.G);
    gv = ld_f(p.g, ((int64_t)bb * p.g_h + hg) * p.g_c + (p.g_c == 1 ? 0 : i), p.g_dt);
    bv = ld_f(p.b, ((int64_t)bb * p.b_h + hb) * p.b_c + (p.b_c == 1 ? 0 : i), p.b_dt);
    wv = ld_f(p.w, ((int64_t)bb * p.w_h + hw) * p.w_c + (p.w_c == 1 ? 0 : i), p.w_dt);
    vv = ld_f(p.v, ((int64_t)bb * p.Hv + hv) * V + i, p.v_dt);
  }
  auto srow = [&](int r) { return sizeof(TSin) == 2 ? 4 * NW * r + rg : R * rg + r; };
  RowIn S[R];
  const TSin* sp = (const TSin*)p.sin + sbase;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (!rst) S[r].load(sp + srow(r) * V, cg);
    else S[r].zero();
  }
  {
    const float sq = wave_sum(xq * xq), sk = wave_sum(xk * xk);
    if (lane == 0 && wid < 2) { rbuf[0][wid] = sq; rbuf[1][wid] = sk; }
  }
  __syncthreads();
  if (tid < 128) {
    float yq, yk;
    if (p.l2norm) {
      yq = xq / sqrtf(rbuf[0][0] + rbuf[0][1] + 1e-6f) * p.scale;
      yk = xk / sqrtf(rbuf[1][0] + rbuf[1][1] + 1e-6f);
    } else {
      yq = xq * p.scale;
      yk = xk;
    }
    float g_ = fminf(gv, 0.f);
    float b_ = bv;
    if (p.guard) { b_ = fmaxf(b_, 0.f); g_ = fminf(g_, -1e-6f); }
    qn[i] = yq;
    kn[i] = yk;
    dd[i] = __expf(g_);
    bt[i] = b_ * yk;
    const float qk = wave_sum(yq * yk);
    if (lane == 0) rbuf[2][wid] = qk;
  }
  __syncthreads();
  const float qk = rbuf[2][0] + rbuf[2][1];

  // this lane's partial column sums of b k^T (D S) and q^T (D S), D = diag(e^g)
  float pa[8], pc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) { pa[e] = 0.f; pc[e] = 0.f; }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int ii = srow(r);
    const float di = dd[ii], bi = bt[ii] * di, qi = qn[ii] * di;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float s = S[r].at(e);
      pa[e] += bi * s;
      pc[e] += qi * s;
    }
  }
  // the 4 row groups of a wave differ in lane bits 4 and 5
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    pa[e] += __shfl_xor(pa[e], 16);
    pa[e] += __shfl_xor(pa[e], 32);
    pc[e] += __shfl_xor(pc[e], 16);
    pc[e] += __shfl_xor(pc[e], 32);
  }
  if (lane < 16) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      red[0][wid][RowIn::col(cg, e)] = pa[e];
      red[1][wid][RowIn::col(cg, e)] = pc[e];
    }
  }
  __syncthreads();
  if (tid < V) {
    const int j = tid;
    float A = 0.f, Cc = 0.f;
#pragma unroll
    for (int r = 0; r < NW; ++r) { A += red[0][r][j]; Cc += red[1][r][j]; }
    const float nv = wv * vv - A;
    vn[j] = nv;
    const float o = Cc + qk * nv;
    const int64_t oi = (int64_t)bh * V + j;
    if (!valid) {
    } else if (p.v_dt == DT_BF16) ((bf16*)p.out)[oi] = (bf16)o;
    else if (p.v_dt == DT_F16) ((f16*)p.out)[oi] = (f16)o;
    else ((float*)p.out)[oi] = o;
  }
  __syncthreads();
  float vc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) vc[e] = vn[RowIn::col(cg, e)];
  // S' = D S + k vn^T, then the optional Frobenius cap
  float fac = 1.f;
  if (p.guard) {
    float ss = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int ii = srow(r);
      const float di = dd[ii], ki = kn[ii];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float y = fmaf(di, S[r].at2(e), ki * vc[e]);
        ss += y * y;
      }
    }
    ss = wave_sum(ss);
    if (lane == 0) gbuf[wid] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) tot += gbuf[w];
    fac = fminf(1.f, p.tau / sqrtf(tot + 1e-6f));
  }
  TSout* op = (TSout*)p.sout + sbase;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int ii = srow(r);
    const float di = dd[ii], ki = kn[ii];
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = fmaf(di, S[r].at2(e), ki * vc[e]) * fac;
    if (valid) store_row<TSin, TSout>(op + srow(r) * V, cg, y);
  }
}

// T consecutive decode steps in one launch: the state stays in registers
// (fp32) across the tokens and is read and written once.  Every step is the
// single-step computation above (its column sums added in another order: 4
// waves of 8 consecutive rows per lane); with a bf16 output state
// the state is rounded to bf16 after every token, as T chained single steps
// would store it.  The per-token LDS vectors are double-buffered by token
// parity, so a token's writes never race the previous token's reads (every
// wave has passed the previous token's barriers before it writes).
template <class TSin, class TSout, int NW>
__global__ __launch_bounds__(64 * NW) void k_decode_multi(const DP p) {
  constexpr int K = 128, V = 128, R = K / (4 * NW);   // rows per lane
  static_assert(NW >= 2 && K % (4 * NW) == 0, "waves per workgroup");
  using RowIn = Row8<TSin>;
  __shared__ float qn[2][K], kn[2][K], dd[2][K], bt[2][K], vn[2][V];
  __shared__ float red[2][2][NW][V];
  __shared__ float rbuf[2][3][2];
  __shared__ float gbuf[2][NW];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wid = tid >> 6;
  const int cg = tid & 15, rg = tid >> 4;
  const int bh = blockIdx.x;
  const int bb = bh / p.Hv, hv = bh % p.Hv;
  const int hk = hv / p.G;
  const int T = p.T;
  const int64_t sbase = (int64_t)bh * K * V;

  // lanes 0-127: element i = tid of q, k, g, b and column j = tid of w, v
  const int i = tid;
  const int hg = dgate_head(p.g_h, p.Hk, p.Hv, hv, p.G);
  const int hb = dgate_head(p.b_h, p.Hk, p.Hv, hv, p.G);
  const int hw = dgate_head(p.w_h, p.Hk, p.Hv, hv, p.G);
  float xq = 0.f, xk = 0.f, gv = 0.f, bv = 0.f, wv = 0.f, vv = 0.f;
  auto ld_tok = [&](int t) {
    if (tid < 128) {
      const int64_t bt_ = (int64_t)bb * T + t;
      const int64_t qo = (bt_ * p.Hk + hk) * K + i;
      xq = ld_f(p.q, qo, p.qk_dt);
      xk = ld_f(p.k, qo, p.qk_dt);
      gv = ld_f(p.g, (bt_ * p.g_h + hg) * p.g_c + (p.g_c == 1 ? 0 : i), p.g_dt);
      bv = ld_f(p.b, (bt_ * p.b_h + hb) * p.b_c + (p.b_c == 1 ? 0 : i), p.b_dt);
      wv = ld_f(p.w, (bt_ * p.w_h + hw) * p.w_c + (p.w_c == 1 ? 0 : i), p.w_dt);
      vv = ld_f(p.v, (bt_ * p.Hv + hv) * V + i, p.v_dt);
    }
  };
  ld_tok(0);   // before the state loads, as in the single step (fp32 state, T = 8: 556 to 514 us)
  float S[R][8];
  {
    const TSin* sp = (const TSin*)p.sin + sbase;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      RowIn raw;
      raw.load(sp + (R * rg + r) * V, cg);
#pragma unroll
      for (int e = 0; e < 8; ++e) S[r][e] = raw.at(e);
    }
  }
#pragma unroll 1
  for (int t = 0; t < T; ++t) {
    const int u = t & 1;
    if (p.reset != nullptr && p.reset[(int64_t)bb * T + t] != 0) {
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int e = 0; e < 8; ++e) S[r][e] = 0.f;
    }
    {
      const float sq = wave_sum(xq * xq), sk = wave_sum(xk * xk);
      if (lane == 0 && wid < 2) { rbuf[u][0][wid] = sq; rbuf[u][1][wid] = sk; }
    }
    __syncthreads();
    if (tid < 128) {
      float yq, yk;
      if (p.l2norm) {
        yq = xq / sqrtf(rbuf[u][0][0] + rbuf[u][0][1] + 1e-6f) * p.scale;
        yk = xk / sqrtf(rbuf[u][1][0] + rbuf[u][1][1] + 1e-6f);
      } else {
        yq = xq * p.scale;
        yk = xk;
      }
      float g_ = fminf(gv, 0.f);
      float b_ = bv;
      if (p.guard) { b_ = fmaxf(b_, 0.f); g_ = fminf(g_, -1e-6f); }
      qn[u][i] = yq;
      kn[u][i] = yk;
      dd[u][i] = __expf(g_);
      bt[u][i] = b_ * yk;
      const float qk = wave_sum(yq * yk);
      if (lane == 0) rbuf[u][2][wid] = qk;
    }
    const float wv_t = wv, vv_t = vv;
    if (t + 1 < T) ld_tok(t + 1);   // the next token's inputs load meanwhile
    __syncthreads();
    const float qk = rbuf[u][2][0] + rbuf[u][2][1];

    float pa[8], pc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) { pa[e] = 0.f; pc[e] = 0.f; }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int ii = R * rg + r;
      const float di = dd[u][ii], bi = bt[u][ii] * di, qi = qn[u][ii] * di;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pa[e] += bi * S[r][e];
        pc[e] += qi * S[r][e];
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      pa[e] += __shfl_xor(pa[e], 16);
      pa[e] += __shfl_xor(pa[e], 32);
      pc[e] += __shfl_xor(pc[e], 16);
      pc[e] += __shfl_xor(pc[e], 32);
    }
    if (lane < 16) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        red[u][0][wid][RowIn::col(cg, e)] = pa[e];
        red[u][1][wid][RowIn::col(cg, e)] = pc[e];
      }
    }
    __syncthreads();
    if (tid < V) {
      const int j = tid;
      float A = 0.f, Cc = 0.f;
#pragma unroll
      for (int r = 0; r < NW; ++r) { A += red[u][0][r][j]; Cc += red[u][1][r][j]; }
      const float nv = wv_t * vv_t - A;
      vn[u][j] = nv;
      const float o = Cc + qk * nv;
      const int64_t oi = (((int64_t)bb * T + t) * p.Hv + hv) * V + j;
      if (p.v_dt == DT_BF16) ((bf16*)p.out)[oi] = (bf16)o;
      else if (p.v_dt == DT_F16) ((f16*)p.out)[oi] = (f16)o;
      else ((float*)p.out)[oi] = o;
    }
    __syncthreads();
    float vc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) vc[e] = vn[u][RowIn::col(cg, e)];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int ii = R * rg + r;
      const float di = dd[u][ii], ki = kn[u][ii];
#pragma unroll
      for (int e = 0; e < 8; ++e) S[r][e] = fmaf(di, S[r][e], ki * vc[e]);
    }
    if (p.guard) {
      float ss = 0.f;
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += S[r][e] * S[r][e];
      ss = wave_sum(ss);
      if (lane == 0) gbuf[u][wid] = ss;
      __syncthreads();
      float tot = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) tot += gbuf[u][w];
      const float fac = fminf(1.f, p.tau / sqrtf(tot + 1e-6f));
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int e = 0; e < 8; ++e) S[r][e] *= fac;
    }
    if constexpr (sizeof(TSout) == 2) {
      // the state a bf16 single step would store and the next one load
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int e = 0; e < 8; ++e) S[r][e] = (float)(bf16)S[r][e];
    }
  }
  TSout* op = (TSout*)p.sout + sbase;
#pragma unroll
  for (int r = 0; r < R; ++r) store_row<TSin, TSout>(op + (R * rg + r) * V, cg, S[r]);
}

__global__ __launch_bounds__(256) void k_frob_cap(float* S, int64_t per, float tau) {
  __shared__ float buf[4];
  float* m = S + (int64_t)blockIdx.x * per;
  float ss = 0.f;
  for (int64_t i = threadIdx.x; i < per; i += 256) ss += m[i] * m[i];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  if ((threadIdx.x & 63) == 0) buf[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float tot = buf[0] + buf[1] + buf[2] + buf[3];
  const float fac = fminf(1.f, tau / sqrtf(tot + 1e-6f));
  for (int64_t i = threadIdx.x; i < per; i += 256) m[i] *= fac;
}

}  // namespace dn

using namespace dn;

extern "C" const char* dn_last_error(void) { return g_last_error.c_str(); }

extern "C" int dn_profile_begin(void) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  g_recs.clear();
  g_prof.store(true);
  return DN_OK;
}

extern "C" int dn_profile_end(double* ms_sum, int64_t* launches) {
  std::vector<ProfRec> recs;
  {
    std::lock_guard<std::mutex> lk(g_prof_mu);
    g_prof.store(false);
    recs.swap(g_recs);
  }
  for (int k = 0; k < DN_PROFILE_KINDS; ++k) {
    if (ms_sum) ms_sum[k] = 0.0;
    if (launches) launches[k] = 0;
  }
  int rc = DN_OK;
  for (const ProfRec& r : recs) {
    float ms = 0.f;
    if (hipEventSynchronize(r.b) != hipSuccess || hipEventElapsedTime(&ms, r.a, r.b) != hipSuccess) {
      rc = set_error(DN_E_LAUNCH, "profiling event failed");
    } else if (r.kind >= 0 && r.kind < DN_PROFILE_KINDS) {
      if (ms_sum) ms_sum[r.kind] += ms;
      if (launches) launches[r.kind] += 1;
    }
  }
  std::lock_guard<std::mutex> lk(g_prof_mu);
  for (const ProfRec& r : recs) {
    g_pool.push_back(r.a);
    g_pool.push_back(r.b);
  }
  return rc;
}

extern "C" int dn_abi_version(void) { return DN_ABI_VERSION; }

namespace {
int decode_launch(const dn_decode_args* a, int T, void* stream) {
  if (a == nullptr) return set_error(DN_E_INVALID, "null args");
  if (a->abi_version != DN_ABI_VERSION) return set_error(DN_E_ABI, "dn_decode_args built for another ABI version");
  if (a->K != 128 || a->V != 128) return set_error(DN_E_INVALID, "K and V must both be 128");
  if (a->B <= 0 || a->Hk <= 0 || a->Hv <= 0 || a->Hv % a->Hk) return set_error(DN_E_INVALID, "bad head counts");
  if (T <= 0) return set_error(DN_E_INVALID, "T must be positive");
  if (!a->q || !a->k || !a->v || !a->g || !a->b || !a->w || !a->state_in || !a->state_out || !a->out)
    return set_error(DN_E_INVALID, "missing tensor pointer");
  auto gate_ok = [&](int H, int Cc, int dt) {
    return (H == 1 || H == a->Hk || H == a->Hv) && (Cc == 1 || Cc == 128) && dt >= DN_F32 && dt <= DN_F16;
  };
  if (!gate_ok(a->g_heads, a->g_chans, a->g_dtype) || !gate_ok(a->b_heads, a->b_chans, a->b_dtype) ||
      !gate_ok(a->w_heads, a->w_chans, a->w_dtype))
    return set_error(DN_E_INVALID, "gate shape/dtype not supported");
  const bool in_ok = a->state_in_dtype == DN_F32 || a->state_in_dtype == DN_BF16;
  const bool out_ok = a->state_out_dtype == DN_F32 || a->state_out_dtype == DN_BF16;
  if (!in_ok || !out_ok) return set_error(DN_E_INVALID, "state dtype must be f32 or bf16");
  if (a->state_in == a->state_out && a->state_in_dtype != a->state_out_dtype)
    return set_error(DN_E_INVALID, "in-place state update needs equal dtypes");
  DP p{};
  p.B = a->B; p.Hk = a->Hk; p.Hv = a->Hv; p.G = a->Hv / a->Hk;
  p.q = a->q; p.k = a->k; p.v = a->v; p.qk_dt = a->qk_dtype; p.v_dt = a->v_dtype;
  p.g = a->g; p.g_dt = a->g_dtype; p.g_h = a->g_heads; p.g_c = a->g_chans;
  p.b = a->b; p.b_dt = a->b_dtype; p.b_h = a->b_heads; p.b_c = a->b_chans;
  p.w = a->w; p.w_dt = a->w_dtype; p.w_h = a->w_heads; p.w_c = a->w_chans;
  p.sin = a->state_in; p.sout = a->state_out; p.reset = a->reset; p.out = a->out;
  p.scale = a->scale; p.l2norm = a->qk_l2norm; p.guard = a->stability_guard; p.tau = a->stability_tau;
  p.T = T;
  hipStream_t st = (hipStream_t)stream;
  const bool fi = a->state_in_dtype == DN_F32, fo = a->state_out_dtype == DN_F32;
  const dim3 grid((unsigned)(a->B * a->Hv));
  // the single-step kernel runs two matrices per workgroup (measured faster at
  // config 4 than one: fp32 state 179 vs 187 us, bf16 state 94 vs 95 us)
  const dim3 grid2((unsigned)((a->B * a->Hv + 1) / 2)), blk2(128 * kDecodeWaves);
  prof_mark(3, st, false);
  if (T == 1) {
    if (fi && fo) hipLaunchKernelGGL((k_decode<float, float, kDecodeWaves, 2>), grid2, blk2, 0, st, p);
    else if (fi && !fo) hipLaunchKernelGGL((k_decode<float, bf16, kDecodeWaves, 2>), grid2, blk2, 0, st, p);
    else if (fo) hipLaunchKernelGGL((k_decode<bf16, float, kDecodeWaves, 2>), grid2, blk2, 0, st, p);
    else hipLaunchKernelGGL((k_decode<bf16, bf16, kDecodeWaves, 2>), grid2, blk2, 0, st, p);
  } else {
    if (fi && fo) hipLaunchKernelGGL((k_decode_multi<float, float, kMultiWaves>), grid, dim3(64 * kMultiWaves), 0, st, p);
    else if (fi && !fo) hipLaunchKernelGGL((k_decode_multi<float, bf16, kMultiWaves>), grid, dim3(64 * kMultiWaves), 0, st, p);
    else if (fo) hipLaunchKernelGGL((k_decode_multi<bf16, float, kMultiWaves>), grid, dim3(64 * kMultiWaves), 0, st, p);
    else hipLaunchKernelGGL((k_decode_multi<bf16, bf16, kMultiWaves>), grid, dim3(64 * kMultiWaves), 0, st, p);
  }
  prof_mark(3, st, true);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(DN_E_LAUNCH, hipGetErrorString(e));
  return DN_OK;
}
}  // namespace

extern "C" int dn_decode_step(const dn_decode_args* a, void* stream) { return decode_launch(a, 1, stream); }

extern "C" int dn_decode_steps(const dn_decode_args* a, int32_t T, void* stream) {
  return decode_launch(a, T, stream);
}

extern "C" int dn_state_frob_cap(float* state, int64_t nmat, int32_t rows, int32_t cols, float tau, void* stream) {
  if (state == nullptr || nmat <= 0 || rows <= 0 || cols <= 0) return set_error(DN_E_INVALID, "bad cap arguments");
  if (!(tau > 0.f)) return set_error(DN_E_INVALID, "tau must be positive");
  hipLaunchKernelGGL(k_frob_cap, dim3((unsigned)nmat), dim3(256), 0, (hipStream_t)stream, state, (int64_t)rows * cols, tau);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(DN_E_LAUNCH, hipGetErrorString(e));
  return DN_OK;
}
