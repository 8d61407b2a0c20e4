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

// One row (elems elements) of a run-time-typed tensor, base t + row * elems
// elements, read through a buffer resource: loads are bounds-checked by the
// hardware (bytes past the row's last whole word read as 0).  Buffer loads
// need 4-byte-aligned addresses, so the resource starts at the word holding
// the row's first byte (o0: the row's offset in it) and a 16-bit element is
// the half of its aligned word that ld_row shifts down.  Loads of a run-time
// type through typed pointers sit in branches whose joins make the compiler
// wait for each load before issuing the next; these do not.  The row must
// stay under 2^31 bytes.
struct TRow {
  __amdgpu_buffer_rsrc_t rs;
  int o0;
};
__device__ __forceinline__ TRow row_rsrc(const void* t, int64_t row, int elems, int dt) {
  const int64_t bytes = (int64_t)elems * (dt == DT_F32 ? 4 : 2);
  const uintptr_t start = reinterpret_cast<uintptr_t>(t) + row * bytes;
  const int o0 = (int)(start & 3);
  // word 3: the gfx9 raw-buffer format (32-bit data, no swizzle)
  return TRow{__builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(start - o0), (short)0,
                                                (int)((o0 + bytes + 3) & ~(int64_t)3), 0x00020000),
              o0};
}
// element idx of such a row as raw bits in the low word (f32) or half word
// (bf16, f16), converted by bits_f once a batch of loads is issued
__device__ __forceinline__ uint32_t ld_row(const TRow& r, int idx, int dt) {
  const int bo = r.o0 + idx * (dt == DT_F32 ? 4 : 2);
  return __builtin_amdgcn_raw_buffer_load_b32(r.rs, bo & ~3, 0, 0) >> (8 * (bo & 2));
}

// raw bits of an element (f32: the word; bf16 and f16: the low half word) as a float
__device__ __forceinline__ float bits_f(uint32_t r, int dt) {
  if (dt == DT_F32) return __builtin_bit_cast(float, r);
  if (dt == DT_BF16) return __builtin_bit_cast(float, r << 16);
  return (float)__builtin_bit_cast(f16, (uint16_t)r);
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

// waves per matrix of the single-step kernel with an fp32 state on either
// side: 2 (16 state rows per lane), two matrices per workgroup (config 4:
// 179 us against 184-192 for 4 waves or other matrix counts).  A bf16 state
// both ways runs 4 waves on one matrix (see the launch).
constexpr int kDecodeWaves = 2;
constexpr int kMultiWaves = 4;   // waves per workgroup of the T-token kernel, fp32 state (8 measured slower)
// launches of at least this many tokens (and no stability guard) run the
// chunked kernel: at config 4 a launch below 16 tokens costs about what one of
// 8 does (212 us bf16 state, 354 us fp32), so it is faster from 6 tokens (per
// token kernel at T = 6: 253 / 377 us, at T = 5: 221 / 338 us)
constexpr int kChunkMinTokens = 6;

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
  // (wave-uniform: the row resources below live in scalar registers)
  const int bh = __builtin_amdgcn_readfirstlane(valid ? bh_raw : p.B * p.Hv - 1);
  const int bb = bh / p.Hv, hv = bh % p.Hv;
  const int hk = hv / p.G;
  const int64_t sbase = (int64_t)bh * K * V;

  // lanes 0-127: element i = tid of q, k, g, b and column j = tid of w, v,
  // every load issued before the first use of any (no branch between them)
  const int i = tid;
  uint32_t xq_ = 0, xk_ = 0, gv_ = 0, bv_ = 0, wv_ = 0, vv_ = 0;
  int rflag = 0;
  if (p.reset != nullptr) rflag = p.reset[bb];
  if (tid < 128) {
    const int hg = dgate_head(p.g_h, p.Hk, p.Hv, hv, p.G);
    const int hb = dgate_head(p.b_h, p.Hk, p.Hv, hv, p.G);
    const int hw = dgate_head(p.w_h, p.Hk, p.Hv, hv, p.G);
    const auto rq = row_rsrc(p.q, bb, p.Hk * K, p.qk_dt), rk = row_rsrc(p.k, bb, p.Hk * K, p.qk_dt);
    const auto rg_ = row_rsrc(p.g, bb, p.g_h * p.g_c, p.g_dt), rb_ = row_rsrc(p.b, bb, p.b_h * p.b_c, p.b_dt);
    const auto rw = row_rsrc(p.w, bb, p.w_h * p.w_c, p.w_dt), rv = row_rsrc(p.v, bb, p.Hv * V, p.v_dt);
    xq_ = ld_row(rq, hk * K + i, p.qk_dt);
    xk_ = ld_row(rk, hk * K + i, p.qk_dt);
    gv_ = ld_row(rg_, hg * p.g_c + (p.g_c == 1 ? 0 : i), p.g_dt);
    bv_ = ld_row(rb_, hb * p.b_c + (p.b_c == 1 ? 0 : i), p.b_dt);
    wv_ = ld_row(rw, hw * p.w_c + (p.w_c == 1 ? 0 : i), p.w_dt);
    vv_ = ld_row(rv, hv * V + i, p.v_dt);
  }
  // the state is loaded whatever the reset flag says (a reset row reads it
  // for nothing) and cleared once the flag is known, so no load waits for it
  auto srow = [&](int r) { return sizeof(TSin) == 2 ? 4 * NW * r + rg : R * rg + r; };
  RowIn S[R];
  const TSin* sp = (const TSin*)p.sin + sbase;
#pragma unroll
  for (int r = 0; r < R; ++r) S[r].load(sp + srow(r) * V, cg);
  // first use of the small loads: only now, after the state loads are issued
  // (an empty asm that "updates" them keeps their conversion from moving up)
  asm volatile("" : "+v"(xq_), "+v"(xk_), "+v"(gv_), "+v"(bv_), "+v"(wv_), "+v"(vv_), "+v"(rflag));
  const bool rst = __builtin_amdgcn_readfirstlane(rflag) != 0;
  const float xq = bits_f(xq_, p.qk_dt), xk = bits_f(xk_, p.qk_dt), gv = bits_f(gv_, p.g_dt),
              bv = bits_f(bv_, p.b_dt), wv = bits_f(wv_, p.w_dt), vv = bits_f(vv_, p.v_dt);
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

  if (rst) {
#pragma unroll
    for (int r = 0; r < R; ++r) S[r].zero();
  }
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
// across the tokens and is read and written once; with a bf16 output state it
// is rounded to bf16 after every token, as T chained single steps would store
// it.  Every step is the single-step computation above (its column sums added in another order: 4 waves of 8
// consecutive rows per lane).  It serves launches with the stability guard
// (the cap applies after every token) and launches of fewer than
// kChunkMinTokens tokens; the others run k_decode_chunk.  The per-token LDS
// vectors are double-buffered by token parity, so a token's writes never race
// the previous token's reads (every wave has passed the previous token's
// barriers before it writes).
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
  // a token's inputs as raw bits (and its reset flag), converted at the top
  // of its step: no load of the batch waits for another
  uint32_t xq_ = 0, xk_ = 0, gv_ = 0, bv_ = 0, wv_ = 0, vv_ = 0;
  int rf_ = 0;
  auto ld_tok = [&](int t) {
    const int64_t row = (int64_t)bb * T + t;
    if (p.reset != nullptr) rf_ = p.reset[row];
    if (tid < 128) {
      const TRow rq = row_rsrc(p.q, row, p.Hk * K, p.qk_dt), rk = row_rsrc(p.k, row, p.Hk * K, p.qk_dt);
      const TRow rg_ = row_rsrc(p.g, row, p.g_h * p.g_c, p.g_dt), rb_ = row_rsrc(p.b, row, p.b_h * p.b_c, p.b_dt);
      const TRow rw = row_rsrc(p.w, row, p.w_h * p.w_c, p.w_dt), rv = row_rsrc(p.v, row, p.Hv * V, p.v_dt);
      xq_ = ld_row(rq, hk * K + i, p.qk_dt);
      xk_ = ld_row(rk, hk * K + i, p.qk_dt);
      gv_ = ld_row(rg_, hg * p.g_c + (p.g_c == 1 ? 0 : i), p.g_dt);
      bv_ = ld_row(rb_, hb * p.b_c + (p.b_c == 1 ? 0 : i), p.b_dt);
      wv_ = ld_row(rw, hw * p.w_c + (p.w_c == 1 ? 0 : i), p.w_dt);
      vv_ = ld_row(rv, hv * V + i, p.v_dt);
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
    // (an empty asm that "updates" the raw inputs keeps their conversion, and
    // so the wait for them, after every load issued before this point)
    asm volatile("" : "+v"(xq_), "+v"(xk_), "+v"(gv_), "+v"(bv_), "+v"(wv_), "+v"(vv_), "+v"(rf_));
    const float xq = bits_f(xq_, p.qk_dt), xk = bits_f(xk_, p.qk_dt), gv = bits_f(gv_, p.g_dt),
                bv = bits_f(bv_, p.b_dt), wv = bits_f(wv_, p.w_dt), vv = bits_f(vv_, p.v_dt);
    if (__builtin_amdgcn_readfirstlane(rf_) != 0) {
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
      const float nv = wv * vv - A;
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
      // the state a bf16 single step would store and the next one load (the
      // compiler then keeps it packed: T = 16, bf16 state 728 us against
      // 922 us with an fp32 carry)
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

// ---------------------------------------------------------------------------
// T consecutive decode steps as chunks of 16 tokens in the chunked WY form
// (the prefill's decomposition with 16-token chunks, the caller's state as
// the state entering the first chunk), for launches without the stability
// guard.  Per chunk of one (batch row, value head), with L the per-channel
// cumulative log-decay inside the chunk and the documents that the reset
// flags start (a reset at token t clears the state before token t):
//   A[t][s] = sum_c b_tc k_tc k_sc e^{L_tc - L_sc}   (t > s, same document)
//   M[t][s] = sum_c q_tc k_sc e^{L_tc - L_sc}        (t >= s, same document)
//   Tm = (I + A)^-1,  W = Tm (b k e^L)_first,  U = Tm (w v)
//   Vn = U - W S,  O = (q e^L)_first S + M Vn,  S <- D S + (k e^{L_end - L})_last^T Vn
// (D = e^{L_end}, or 0 when the chunk holds a reset), which is the
// token-by-token recurrence (gdn2.py:2471-2478) in exact arithmetic.  The
// 16-row products run on MFMA in split bf16 (hi / lo words, 3 products), so
// the state is read and written once per launch and a token costs a share of
// a few 16-row products instead of three passes over the state.  The state
// stays fp32 (MFMA accumulators) across the T tokens and is rounded to the
// output state type once, at the end.
// Layout: 4 waves; wave w owns state columns 32w..32w+31 as accumulator tiles
// S[rt][ct] (lane (c, q): rows 16rt + 4q + ii of column 32w + 16ct + c), and
// two stacked row tiles are the B operand of one 32-row slab, so no
// reduction crosses waves.  The chunk's 16 x 128 operands are formed in LDS
// by all 256 threads.  The state moves between row-major memory and the
// accumulator layout through identity products (exact), never through LDS.
// ---------------------------------------------------------------------------
// An element of a run-time-typed tensor as raw bits (f32: the word; bf16 and
// f16: the half word), converted after every load of a batch is issued: a
// conversion inside the type branch would wait for each load in turn.
__device__ __forceinline__ uint32_t ld_bits(const void* p, int64_t i, int dt) {
  if (dt == DT_F32) return ((const uint32_t*)p)[i];
  return ((const uint16_t*)p)[i];
}

// Sum over the 16 lanes of a DPP row, every lane receiving the same value:
// quad swaps, then rotations by 8 and by 4, an order in which all 16 lanes
// add the same pairs (bit-identical totals).
template <int C> __device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), C, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp<0xB1>(x);    // quad_perm [1, 0, 3, 2]
  x += dpp<0x4E>(x);    // quad_perm [2, 3, 0, 1]
  x += dpp<0x128>(x);   // row_ror:8
  x += dpp<0x124>(x);   // row_ror:4
  return x;
}

// 8 consecutive elements of a run-time-typed tensor as raw 16-byte words (f32:
// two, 16-bit types: one), converted after every load of a batch is issued.
struct Raw8w { uint4 a, b; };
__device__ __forceinline__ void ld8_bits(const void* p, int64_t i, int dt, Raw8w& r) {
  if (dt == DT_F32) {
    r.a = *reinterpret_cast<const uint4*>((const float*)p + i);
    r.b = *reinterpret_cast<const uint4*>((const float*)p + i + 4);
  } else {
    r.a = *reinterpret_cast<const uint4*>((const uint16_t*)p + i);
    r.b = r.a;
  }
}
__device__ __forceinline__ void bits8_f(const Raw8w& r, int dt, float* x) {
  const uint32_t wa[4] = {r.a.x, r.a.y, r.a.z, r.a.w}, wb[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
  if (dt == DT_F32) {
#pragma unroll
    for (int e = 0; e < 4; ++e) { x[e] = __builtin_bit_cast(float, wa[e]); x[4 + e] = __builtin_bit_cast(float, wb[e]); }
  } else if (dt == DT_BF16) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = __builtin_bit_cast(float, wa[e] << 16);
      x[2 * e + 1] = __builtin_bit_cast(float, wa[e] & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = (float)__builtin_bit_cast(f16, (uint16_t)(wa[e] & 0xffffu));
      x[2 * e + 1] = (float)__builtin_bit_cast(f16, (uint16_t)(wa[e] >> 16));
    }
  }
}

constexpr int DC = 16;      // tokens per chunk
constexpr int DCP = 132;    // fp32 pitch of the [token][channel] LDS arrays
constexpr int AP = 20;      // fp32 pitch of the 16 x 16 token-pair arrays (16-byte rows)

// An fp32 fragment as three bf16 fragments whose sum is exactly x (8
// significant bits each: the remainders after each rounding are exact in
// fp32 and the last fits a bf16), so identity products on the bf16 MFMA
// move fp32 values between layouts exactly.
__device__ __forceinline__ void split3(const float* x, Frag<true>& a, Frag<true>& b, Frag<true>& c) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const bf16 h = (bf16)x[e];
    const float r1 = x[e] - (float)h;
    const bf16 m = (bf16)r1;
    a.v[e] = h;
    b.v[e] = m;
    c.v[e] = (bf16)(r1 - (float)m);
  }
}

// decay span (nats) up to which a chunk's A and M are formed as products of
// per-token factors e^{L_t - L_8}, e^{L_8 - L_s} (each within e^{+-80}, far
// inside the fp32 range); wider chunks take one exponential per pair
constexpr float kChunkSpan = 80.f;

// GK: every gate is fp32 with one value per channel (the gate loads then
// carry no branch on the type or the channel count, which would make the
// compiler wait for each load in turn)
template <class TSin, class TSout, bool BF, bool GK>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_decode_chunk(const DP p) {
  constexpr int K = 128, V = 128;
  using P = Pol<BF>;
  using F3 = typename P::F3;
  __shared__ __align__(16) float lds[9 * DC * DCP + 2 * DC * AP + K + 3 * DC];
  float* sQ = lds;                  // q                                [DC][DCP]
  float* sK = sQ + DC * DCP;        // k
  float* sB = sK + DC * DCP;        // b k
  float* sL = sB + DC * DCP;        // g -> L (high word) -> A / M partial sums -> W
  float* sLl = sL + DC * DCP;       // L (low word) -> U^T [V][DC]
  float* sV = sLl + DC * DCP;       // w v
  float* sBe = sV + DC * DCP;       // (b k e^L)_first
  float* sQe = sBe + DC * DCP;      // (q e^L)_first
  float* sKe = sQe + DC * DCP;      // (k e^{L_end - L})_last, transposed [K][DC]
  // bf16 mode keeps -W, (q e^L)_first and ke^T as split bf16 planes (high
  // words, then low words) in the space of their fp32 arrays, split once by
  // the thread that forms them rather than by every wave that reads them
  bf16* sWh = reinterpret_cast<bf16*>(sL);   // -W   [DC][DCP] high, then low
  bf16* sQh = reinterpret_cast<bf16*>(sQe);  // q e^L
  bf16* sKh = reinterpret_cast<bf16*>(sKe);  // ke^T [K][DC]
  constexpr int WPL = DC * DCP;              // bf16 offset of a low plane
  constexpr int KPL = K * DC;
  float* sA = sKe + DC * DCP;       // A   [DC][DC + 1]
  float* sM = sA + DC * AP;   // M
  float* sD = sM + DC * AP;   // state row factor of the chunk
  int* sDoc = reinterpret_cast<int*>(sD + K);   // [0, DC): document of token t; [DC, 2DC): reset flags
  int* sWide = sDoc + 2 * DC;                    // a channel's decay span exceeds kChunkSpan

  const int tid = threadIdx.x;
  const int l = tid & 63, w = tid >> 6, r16 = l & 15, q = l >> 4;
  const int bh = blockIdx.x;
  const int bb = bh / p.Hv, hv = bh % p.Hv;
  const int hk = hv / p.G;
  const int T = p.T;
  const int64_t sbase = (int64_t)bh * K * V;
  const int hg = dgate_head(p.g_h, p.Hk, p.Hv, hv, p.G);
  const int hb = dgate_head(p.b_h, p.Hk, p.Hv, hv, p.G);
  const int hw = dgate_head(p.w_h, p.Hk, p.Hv, hv, p.G);

  // token rows of a chunk as raw words: thread (t = tid >> 4, channels
  // 8 (tid & 15) ..+7) loads token t's segment of q, k, v and the gates
  // (tokens past the end read the last one; zeroed later)
  struct Tok { Raw8w q, k, v, g, b, w; int rst; };
  const int tr_t = tid >> 4, c8 = 8 * (tid & 15);
  auto issue_tok = [&](int tb, Tok& r) {
    const int tt = min(tb + tr_t, T - 1);
    const int64_t bt_ = (int64_t)bb * T + tt;
    ld8_bits(p.q, (bt_ * p.Hk + hk) * K + c8, p.qk_dt, r.q);
    ld8_bits(p.k, (bt_ * p.Hk + hk) * K + c8, p.qk_dt, r.k);
    ld8_bits(p.v, (bt_ * p.Hv + hv) * V + c8, p.v_dt, r.v);
    auto gate = [&](const void* g, int H, int C, int dt, int hh, Raw8w& o) {
      if constexpr (GK) {
        const float* gp = (const float*)g + (bt_ * H + hh) * K + c8;
        o.a = *reinterpret_cast<const uint4*>(gp);
        o.b = *reinterpret_cast<const uint4*>(gp + 4);
        return;
      }
      if (C == 1) {
        o.a.x = ld_bits(g, bt_ * H + hh, dt);
        o.b = o.a;
      } else {
        ld8_bits(g, (bt_ * H + hh) * C + c8, dt, o);
      }
    };
    gate(p.g, p.g_h, p.g_c, p.g_dt, hg, r.g);
    gate(p.b, p.b_h, p.b_c, p.b_dt, hb, r.b);
    gate(p.w, p.w_h, p.w_c, p.w_dt, hw, r.w);
    r.rst = 0;
    if (p.reset != nullptr && (tid & 15) == 0) r.rst = p.reset[(int64_t)bb * T + tt];
  };
  Tok tok;
  issue_tok(0, tok);   // chunk 0's rows first: vmcnt retires loads in issue order
  // ---- state in, without LDS: each 16-row tile of the wave's 32 columns is
  // loaded as an A fragment (lane (r16, q): row 16rt + r16, columns
  // 32w + pi(q, 0..7)); its products with the two halves of a 32 x 32 identity
  // are the accumulator tiles S[rt][0], S[rt][1] (exact; an fp32 state as
  // three bf16 parts).  The loads are issued after chunk 0's token rows
  // (so a wait for a row does not wait for the state) and consumed only after
  // chunk 0's token phases, so their latency and the token rows' overlap.
  typedef typename std::conditional<sizeof(TSin) == 2, bf16x4, f32x4>::type RawS;
  RawS ra[8], rb[8];
  {
    const TSin* sp = (const TSin*)p.sin + sbase + 32 * w + 4 * q;
#pragma unroll
    for (int rt = 0; rt < 8; ++rt) {
      const TSin* rp = sp + (int64_t)(16 * rt + r16) * V;
      ra[rt] = *reinterpret_cast<const RawS*>(rp);
      rb[rt] = *reinterpret_cast<const RawS*>(rp + 16);
    }
  }
  f32x4 S[8][2];
  auto state_in = [&]() {
    const Frag<true> id0 = ident_frag<true>(0, r16, q), id1 = ident_frag<true>(1, r16, q);
#pragma unroll
    for (int rt = 0; rt < 8; ++rt) {
      const float x[8] = {(float)ra[rt][0], (float)ra[rt][1], (float)ra[rt][2], (float)ra[rt][3],
                          (float)rb[rt][0], (float)rb[rt][1], (float)rb[rt][2], (float)rb[rt][3]};
      S[rt][0] = zero4();
      S[rt][1] = zero4();
      if constexpr (sizeof(TSin) == 2) {
        Frag<true> f;   // the stored bf16 values as they are
        f.v = __builtin_shufflevector(ra[rt], rb[rt], 0, 1, 2, 3, 4, 5, 6, 7);
        mma(S[rt][0], f, id0);
        mma(S[rt][1], f, id1);
      } else {
        Frag<true> fa, fb, fc;
        split3(x, fa, fb, fc);
        mma(S[rt][0], fa, id0);
        mma(S[rt][1], fa, id1);
        mma(S[rt][0], fb, id0);
        mma(S[rt][1], fb, id1);
        mma(S[rt][0], fc, id0);
        mma(S[rt][1], fc, id1);
      }
    }
  };

  const int nchunk = (T + DC - 1) / DC;
  // everything of a chunk up to W and U (LDS operands only)
  auto chunk_operands = [&](int c0) {
    const int tb = c0 * DC;
    // ---- token rows: prologue (gdn2.py:2393-2438) into LDS
    {
      const bool ok = tb + tr_t < T;
      float xq[8], xk[8], xv[8], xg[8], xb[8], xw[8];
      bits8_f(tok.q, p.qk_dt, xq);
      bits8_f(tok.k, p.qk_dt, xk);
      bits8_f(tok.v, p.v_dt, xv);
      auto gate = [&](const Raw8w& r, int C, int dt, float* x) {
        if constexpr (GK) {
          bits8_f(r, DT_F32, x);
          return;
        }
        if (C == 1) {
          const float s1 = bits_f(r.a.x, dt);
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] = s1;
        } else {
          bits8_f(r, dt, x);
        }
      };
      gate(tok.g, p.g_c, p.g_dt, xg);
      gate(tok.b, p.b_c, p.b_dt, xb);
      gate(tok.w, p.w_c, p.w_dt, xw);
      float sq = 0.f, sk = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) { sq = fmaf(xq[e], xq[e], sq); sk = fmaf(xk[e], xk[e], sk); }
      sq = row16_sum(sq);
      sk = row16_sum(sk);
      float yq[8], yk[8], yb[8], yg[8], yv[8];
      const float iq = 1.f / sqrtf(sq + 1e-6f), ik = 1.f / sqrtf(sk + 1e-6f);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (p.l2norm) {
          yq[e] = xq[e] * iq * p.scale;
          yk[e] = xk[e] * ik;
        } else {
          yq[e] = xq[e] * p.scale;
          yk[e] = xk[e];
        }
        yq[e] = ok ? yq[e] : 0.f;
        yk[e] = ok ? yk[e] : 0.f;
        yb[e] = ok ? xb[e] * yk[e] : 0.f;
        yg[e] = ok ? fminf(xg[e], 0.f) : 0.f;   // _nonpositive (NaN -> 0)
        yv[e] = ok ? xw[e] * xv[e] : 0.f;
      }
      const int o = tr_t * DCP + c8;
      st4<float>(&sQ[o], yq); st4<float>(&sQ[o + 4], yq + 4);
      st4<float>(&sK[o], yk); st4<float>(&sK[o + 4], yk + 4);
      st4<float>(&sB[o], yb); st4<float>(&sB[o + 4], yb + 4);
      st4<float>(&sL[o], yg); st4<float>(&sL[o + 4], yg + 4);
      st4<float>(&sV[o], yv); st4<float>(&sV[o + 4], yv + 4);
      if ((tid & 15) == 0) sDoc[DC + tr_t] = (ok && tok.rst != 0) ? 1 : 0;
      if (tid == 0) sWide[0] = 0;
    }
    __syncthreads();
    // ---- L per channel (double-float running sum), the documents, and the
    // row factors: thread (channel c = tid & 127, tokens 8h..8h+7, h = tid >> 7);
    // both threads of a channel form the whole sum, each writes its half
    {
      const int c = tid & 127, h = tid >> 7;
      // the running sums and documents of this thread's half only (static
      // register indices: a token belongs to the half under a predicate)
      float Lh[8], Ll[8];
      int doc8[8], d = 0;
      float hi = 0.f, lo = 0.f, g0 = 0.f;
#pragma unroll
      for (int t = 0; t < DC; ++t) {
        const float gv = sL[t * DCP + c];
        if (t == 0) g0 = gv;
        d += sDoc[DC + t];
        const float sum = hi + gv;
        const float bbv = sum - hi;
        lo += (hi - (sum - bbv)) + (gv - bbv);
        hi = sum;
        if ((t >> 3) == h) { Lh[t & 7] = hi; Ll[t & 7] = lo; doc8[t & 7] = d; }
        if (tid == t) sDoc[t] = d;   // (read after the barrier below the factors)
      }
      const int dl = d;
      // L_0 - L_15 >= 0 (g <= 0): the chunk's decay span on this channel
      const bool wide = -(hi + lo) + g0 > kChunkSpan;
      if (__any(wide) && l == 0) sWide[0] = 1;
      if (h == 0) sD[c] = dl == 0 ? __expf(hi + lo) : 0.f;
      __syncthreads();   // both halves have read g
      float ke8[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float lh = Lh[j], ll = Ll[j];
        const int dt = doc8[j];
        const int o = (8 * h + j) * DCP + c;
        sL[o] = lh;
        sLl[o] = ll;
        const float eL = __expf(lh + ll);                     // e^{L_t} <= 1
        const float eK = __expf((hi - lh) + (lo - ll));       // e^{L_end - L_t} <= 1
        sBe[o] = dt == 0 ? sB[o] * eL : 0.f;
        const float qe = dt == 0 ? sQ[o] * eL : 0.f;
        if constexpr (BF) {
          const bf16 hh = (bf16)qe;
          sQh[(8 * h + j) * DCP + c] = hh;
          sQh[WPL + (8 * h + j) * DCP + c] = (bf16)(qe - (float)hh);
        } else {
          sQe[o] = qe;
        }
        ke8[j] = dt == dl ? sK[o] * eK : 0.f;
      }
      // ke^T (row = channel, 16 tokens): the update's A operand is one 16-byte read
      if constexpr (BF) {
        bf16x8 kh, kl;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          kh[j] = (bf16)ke8[j];
          kl[j] = (bf16)(ke8[j] - (float)kh[j]);
        }
        *reinterpret_cast<bf16x8*>(&sKh[c * DC + 8 * h]) = kh;
        *reinterpret_cast<bf16x8*>(&sKh[KPL + c * DC + 8 * h]) = kl;
      } else {
        st4<float>(&sKe[c * DC + 8 * h], ke8);
        st4<float>(&sKe[c * DC + 8 * h + 4], ke8 + 4);
      }
    }
    __syncthreads();
    // ---- A and M
    const bool wide = sWide[0] != 0;
    if (!wide) {
      // factored: A = (b k e^{L - L_8}) (k e^{L_8 - L})^T, M = (q e^{L - L_8}) (k e^{L_8 - L})^T
      // on MFMA: wave w sums over channel slab w (lane (t | s = r16, q)) and
      // leaves its partial A and M in that slab's columns of L, which only it reads
      f32x4 pa = zero4(), pm = zero4();
      {
        const int s2 = w;
        float xb[8], xq[8], kc[8], lr[8], lrl[8], lt[8], ltl[8];
        row8<float>(&sB[r16 * DCP + 32 * s2], q, xb);
        row8<float>(&sQ[r16 * DCP + 32 * s2], q, xq);
        row8<float>(&sK[r16 * DCP + 32 * s2], q, kc);
        row8<float>(&sL[8 * DCP + 32 * s2], q, lr);
        row8<float>(&sLl[8 * DCP + 32 * s2], q, lrl);
        row8<float>(&sL[r16 * DCP + 32 * s2], q, lt);
        row8<float>(&sLl[r16 * DCP + 32 * s2], q, ltl);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = (lt[e] - lr[e]) + (ltl[e] - lrl[e]);   // row r16: L - L_8
          const float ex = __expf(d);
          xb[e] *= ex;
          xq[e] *= ex;
          kc[e] *= __expf(-d);
        }
        const F3 fk = P::f3(kc);
        P::m33(pa, P::f3(xb), fk);   // pa[ii] = (row 4q + ii) . (column r16)
        P::m33(pm, P::f3(xq), fk);
      }
      // partial tile of slab w: A at columns 32w + 0..15, M at 32w + 16..31
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        sL[(4 * q + ii) * DCP + 32 * w + r16] = pa[ii];
        sL[(4 * q + ii) * DCP + 32 * w + 16 + r16] = pm[ii];
      }
      __syncthreads();
      {
        const int t = tid & 15, s2 = tid >> 4;
        float a = 0.f, m = 0.f;
#pragma unroll
        for (int ww = 0; ww < 4; ++ww) {
          a += sL[t * DCP + 32 * ww + s2];
          m += sL[t * DCP + 32 * ww + 16 + s2];
        }
        const bool same = sDoc[t] == sDoc[s2];
        sA[t * AP + s2] = (s2 < t && same) ? a : 0.f;
        sM[t * AP + s2] = (s2 <= t && same) ? m : 0.f;
      }
    } else {
      // one exponential per pair: thread (t = tid & 15, s = tid >> 4)
      const int t = tid & 15, s2 = tid >> 4;
      float a = 0.f, m = 0.f;
      if (s2 <= t && sDoc[t] == sDoc[s2]) {
#pragma unroll 1
        for (int c = 0; c < K; c += 4) {
          const f32x4 lt = *reinterpret_cast<const f32x4*>(&sL[t * DCP + c]);
          const f32x4 ls = *reinterpret_cast<const f32x4*>(&sL[s2 * DCP + c]);
          const f32x4 ltl = *reinterpret_cast<const f32x4*>(&sLl[t * DCP + c]);
          const f32x4 lsl = *reinterpret_cast<const f32x4*>(&sLl[s2 * DCP + c]);
          const f32x4 bt = *reinterpret_cast<const f32x4*>(&sB[t * DCP + c]);
          const f32x4 qt = *reinterpret_cast<const f32x4*>(&sQ[t * DCP + c]);
          const f32x4 ks = *reinterpret_cast<const f32x4*>(&sK[s2 * DCP + c]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float ex = __expf((lt[e] - ls[e]) + (ltl[e] - lsl[e]));   // <= 1
            const float kx = ks[e] * ex;
            a = fmaf(bt[e], kx, a);
            m = fmaf(qt[e], kx, m);
          }
        }
      }
      sA[t * AP + s2] = s2 < t ? a : 0.f;
      sM[t * AP + s2] = m;   // 0 above the diagonal and across documents
    }
    __syncthreads();
    // ---- W and U by forward substitution, (I + A) W = be and (I + A) U = w v:
    // thread tid < 128 solves column tid of W (into sL), the others column
    // tid - 128 of U (into sLl); every thread reads its own column only
    {
      const int c = tid & 127;
      const float* rhs = tid < K ? sBe : sV;
      float x[DC];
#pragma unroll
      for (int t = 0; t < DC; ++t) x[t] = rhs[t * DCP + c];
      // row t + 1's reads are issued before row t's products, so each row's
      // LDS latency overlaps the row before; A is the same for every lane, so
      // a row moves to scalar registers as it is used (no vector registers
      // held for it)
      float an[DC];
      an[0] = sA[1 * AP];
#pragma unroll
      for (int t = 1; t < DC; ++t) {
        float ac[DC];
#pragma unroll
        for (int s2 = 0; s2 < t; ++s2)
          ac[s2] = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, an[s2])));
        if (t + 1 < DC) {
#pragma unroll
          for (int s2 = 0; s2 <= t; ++s2) an[s2] = sA[(t + 1) * AP + s2];
        }
        __builtin_amdgcn_sched_barrier(0);
        float acc = x[t];
#pragma unroll
        for (int s2 = 0; s2 < t; ++s2) acc = fmaf(-ac[s2], x[s2], acc);
        x[t] = acc;
      }
      if (tid < K) {
        if constexpr (BF) {
#pragma unroll
          for (int t = 0; t < DC; ++t) {
            const bf16 hh = (bf16)(-x[t]);
            sWh[t * DCP + c] = hh;
            sWh[WPL + t * DCP + c] = (bf16)(-x[t] - (float)hh);
          }
        } else {
#pragma unroll
          for (int t = 0; t < DC; ++t) sL[t * DCP + c] = x[t];
        }
      } else {
        // U^T (row = value column, 16 tokens): the products' accumulator init is one 16-byte read
#pragma unroll
        for (int t4 = 0; t4 < DC; t4 += 4) st4<float>(&sLl[c * DC + t4], x + t4);
      }
    }
    __syncthreads();
  };
  // the wave's state columns: outputs and the state update
  auto chunk_products = [&](int c0) {
    const int tb = c0 * DC;
    // ---- the wave's 32 state columns: Vn, O, state update
    {
      f32x4 vn[2], o[2];
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        o[ct] = zero4();
        vn[ct] = *reinterpret_cast<const f32x4*>(&sLl[(32 * w + 16 * ct + r16) * DC + 4 * q]);
      }
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2) {
        F3 Sf[2];
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
          const float x[8] = {S[2 * s2][ct][0], S[2 * s2][ct][1], S[2 * s2][ct][2], S[2 * s2][ct][3],
                              S[2 * s2 + 1][ct][0], S[2 * s2 + 1][ct][1], S[2 * s2 + 1][ct][2], S[2 * s2 + 1][ct][3]};
          Sf[ct] = P::f3(x);
        }
        F3 Wf, Qf;
        if constexpr (BF) {
          auto plane8 = [&](const bf16* pl) {
            const bf16* rp = pl + r16 * DCP + 32 * s2 + 4 * q;
            Frag<true> f;
            f.v = __builtin_shufflevector(*reinterpret_cast<const bf16x4*>(rp), *reinterpret_cast<const bf16x4*>(rp + 16),
                                          0, 1, 2, 3, 4, 5, 6, 7);
            return f;
          };
          Wf.hi = plane8(sWh); Wf.lo = plane8(sWh + WPL);
          Qf.hi = plane8(sQh); Qf.lo = plane8(sQh + WPL);
        } else {
          float xw[8], xq[8];
          row8<float>(&sL[r16 * DCP + 32 * s2], q, xw);
          row8<float>(&sQe[r16 * DCP + 32 * s2], q, xq);
#pragma unroll
          for (int e = 0; e < 8; ++e) xw[e] = -xw[e];
          Wf = P::f3(xw);
          Qf = P::f3(xq);
        }
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
          P::m33(vn[ct], Wf, Sf[ct]);   // Vn[4q + ii][col] = U - W S
          P::m33(o[ct], Qf, Sf[ct]);    // (q e^L) S
        }
      }
      // Vn as the B operand (k = token): tokens 4q..4q+3 from the accumulator, 16..31 zero
      F3 Vf[2];
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        const float x[8] = {vn[ct][0], vn[ct][1], vn[ct][2], vn[ct][3], 0.f, 0.f, 0.f, 0.f};
        Vf[ct] = P::f3(x);
      }
      {
        const f32x4 m4 = *reinterpret_cast<const f32x4*>(&sM[r16 * AP + 4 * q]);
        const float xm[8] = {m4[0], m4[1], m4[2], m4[3], 0.f, 0.f, 0.f, 0.f};
        const F3 Mf = P::f3(xm);
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) P::m33(o[ct], Mf, Vf[ct]);
      }
      // outputs: lane (c, q) holds tokens 4q..4q+3 of column 32w + 16ct + c
      // (one 64-bit base per chunk; the chunk's offsets fit 32 bits)
      {
        const int ostr = p.Hv * V;   // elements from one token's row to the next
        const int64_t obase = ((int64_t)bb * T + tb) * ostr + (int64_t)hv * V + 32 * w + r16;
        auto store_out = [&](auto* op) {
#pragma unroll
          for (int ct = 0; ct < 2; ++ct)
#pragma unroll
            for (int ii = 0; ii < 4; ++ii)
              if (tb + 4 * q + ii < T) op[(4 * q + ii) * ostr + 16 * ct] = from_f<std::remove_pointer_t<decltype(op)>>(o[ct][ii]);
        };
        if (p.v_dt == DT_BF16) store_out((bf16*)p.out + obase);
        else if (p.v_dt == DT_F16) store_out((f16*)p.out + obase);
        else store_out((float*)p.out + obase);
      }
      // S <- D S + Ke^T Vn
#pragma unroll
      for (int rt = 0; rt < 8; ++rt) {
        const f32x4 d4 = *reinterpret_cast<const f32x4*>(&sD[16 * rt + 4 * q]);
        F3 Kf;
        if constexpr (BF) {
          const bf16x4 z4 = {};
          const bf16* kp = sKh + (16 * rt + r16) * DC + 4 * q;
          Kf.hi.v = __builtin_shufflevector(*reinterpret_cast<const bf16x4*>(kp), z4, 0, 1, 2, 3, 4, 5, 6, 7);
          Kf.lo.v = __builtin_shufflevector(*reinterpret_cast<const bf16x4*>(kp + KPL), z4, 0, 1, 2, 3, 4, 5, 6, 7);
        } else {
          const f32x4 k4 = *reinterpret_cast<const f32x4*>(&sKe[(16 * rt + r16) * DC + 4 * q]);
          const float xk[8] = {k4[0], k4[1], k4[2], k4[3], 0.f, 0.f, 0.f, 0.f};
          Kf = P::f3(xk);
        }
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) S[rt][ct][ii] *= d4[ii];
          P::m33(S[rt][ct], Kf, Vf[ct]);
        }
      }
    }
    // the next chunk's rows load across the barrier (chunk 0's were issued at entry)
    __builtin_amdgcn_sched_barrier(0);   // (not hoisted into the products above)
    if (c0 + 1 < nchunk) issue_tok(tb + DC, tok);
    __syncthreads();
  };
  chunk_operands(0);
  state_in();
  chunk_products(0);
#pragma unroll 1
  for (int c0 = 1; c0 < nchunk; ++c0) {
    chunk_operands(c0);
    chunk_products(c0);
  }

  // ---- state out, without LDS: the accumulator pair of slab s2 read as an A
  // operand is S^T (row = state column, k = state row); its products with the
  // identity halves give lane (c, q) state row 32 s2 + 16 hf + c, columns
  // 32w + 16ct + 4q .. +3 (a bf16 state is rounded first, an fp32 one moves as
  // three bf16 parts: exact either way).  Plain (cached) loads and stores:
  // each instruction covers 32-byte pieces of 16 rows, which the L2 merges
  // (non-temporal ones measured 20 % slower here).
  {
    TSout* op = (TSout*)p.sout + sbase + 32 * w + 4 * q;
    const Frag<true> id0 = ident_frag<true>(0, r16, q), id1 = ident_frag<true>(1, r16, q);
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2) {
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        const float x[8] = {S[2 * s2][ct][0], S[2 * s2][ct][1], S[2 * s2][ct][2], S[2 * s2][ct][3],
                            S[2 * s2 + 1][ct][0], S[2 * s2 + 1][ct][1], S[2 * s2 + 1][ct][2], S[2 * s2 + 1][ct][3]};
        Frag<true> fa, fb, fc;
        if constexpr (sizeof(TSout) == 2) {
          fa = make_frag<true>(x);   // the stored bf16 state
        } else {
          split3(x, fa, fb, fc);
        }
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          f32x4 y = zero4();
          mma(y, fa, hf ? id1 : id0);
          if constexpr (sizeof(TSout) == 4) {
            mma(y, fb, hf ? id1 : id0);
            mma(y, fc, hf ? id1 : id0);
          }
          TSout* rp = op + (int64_t)(32 * s2 + 16 * hf + r16) * V + 16 * ct;
          if constexpr (sizeof(TSout) == 2) {
            const bf16x4 h{(bf16)y[0], (bf16)y[1], (bf16)y[2], (bf16)y[3]};
            *reinterpret_cast<bf16x4*>(rp) = h;
          } else {
            *reinterpret_cast<f32x4*>(rp) = y;
          }
        }
      }
    }
  }
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
int g_decode_chunk = -1;   // -1: unread; 0: per-token kernel forced (DN_DECODE_CHUNK=0, measurements)
bool decode_chunked() {
  if (g_decode_chunk < 0) {
    const char* e = getenv("DN_DECODE_CHUNK");
    g_decode_chunk = (e && atoi(e) == 0) ? 0 : 1;
  }
  return g_decode_chunk == 1;
}

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
    // a bf16 state both ways: four waves on one matrix per workgroup (90.4-90.8
    // vs 91.1-91.4 us at config 4; the fp32 forms measured slower so: 184 vs 179)
    else hipLaunchKernelGGL((k_decode<bf16, bf16, 4, 1>), grid, dim3(256), 0, st, p);
  } else if (!p.guard && T >= kChunkMinTokens && decode_chunked()) {
    // products on the fp32 MFMA when either side of the state is fp32, in
    // split bf16 for a bf16 state (its rounding dominates)
    const bool gk = a->g_dtype == DN_F32 && a->b_dtype == DN_F32 && a->w_dtype == DN_F32 && a->g_chans == 128 &&
                    a->b_chans == 128 && a->w_chans == 128;
    if (fi && fo) {
      if (gk) hipLaunchKernelGGL((k_decode_chunk<float, float, false, true>), grid, dim3(256), 0, st, p);
      else hipLaunchKernelGGL((k_decode_chunk<float, float, false, false>), grid, dim3(256), 0, st, p);
    } else if (fi && !fo) {
      if (gk) hipLaunchKernelGGL((k_decode_chunk<float, bf16, false, true>), grid, dim3(256), 0, st, p);
      else hipLaunchKernelGGL((k_decode_chunk<float, bf16, false, false>), grid, dim3(256), 0, st, p);
    } else if (fo) {
      if (gk) hipLaunchKernelGGL((k_decode_chunk<bf16, float, false, true>), grid, dim3(256), 0, st, p);
      else hipLaunchKernelGGL((k_decode_chunk<bf16, float, false, false>), grid, dim3(256), 0, st, p);
    } else {
      if (gk) hipLaunchKernelGGL((k_decode_chunk<bf16, bf16, true, true>), grid, dim3(256), 0, st, p);
      else hipLaunchKernelGGL((k_decode_chunk<bf16, bf16, true, false>), grid, dim3(256), 0, st, p);
    }
  } else {
    if (fi && fo) hipLaunchKernelGGL((k_decode_multi<float, float, kMultiWaves>), grid, dim3(64 * kMultiWaves), 0, st, p);
    else if (fi && !fo) hipLaunchKernelGGL((k_decode_multi<float, bf16, kMultiWaves>), grid, dim3(64 * kMultiWaves), 0, st, p);
    else if (fo) hipLaunchKernelGGL((k_decode_multi<bf16, float, kMultiWaves>), grid, dim3(64 * kMultiWaves), 0, st, p);
    // a bf16 state both ways: two waves per matrix (T = 4: 188-192 vs 216-219
    // us at config 4; the fp32 forms measured slower so: 327 vs 292)
    else hipLaunchKernelGGL((k_decode_multi<bf16, bf16, 2>), grid, dim3(128), 0, st, p);
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
