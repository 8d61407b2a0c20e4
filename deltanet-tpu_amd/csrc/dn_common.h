// Shared device helpers for the gfx950 delta-rule kernels.
//
// Fragment convention used by every MFMA in this library
// ------------------------------------------------------
// All matrix products are 16x16 output tiles reduced over 32-wide k slabs.
// A lane l of a 64-wide wavefront owns index (l & 15) of the tile's row (A
// operand) or column (B operand) and 8 k values of the slab, chosen by its
// lane group q = l >> 4 through the permutation
//
//     pi(q, e) = 4q + e          (e = 0..3)
//     pi(q, e) = 16 + 4q + e-4   (e = 4..7)
//
// With this permutation the 16x16 fp32 accumulator tile (lane l holds column
// l&15, rows 4q..4q+3) of two vertically stacked tiles IS a B-operand
// fragment of the next product, so chained products (U - W*S, M*Vnew,
// ke^T*Vnew ...) need no LDS round trip.  The same fragment feeds
//   * v_mfma_f32_16x16x32_bf16 (one instruction, 8 bf16 per lane), or
//   * 8 x v_mfma_f32_16x16x4_f32 (step e uses k slot q <-> pi(q, e)),
// so the bf16 and fp32 precisions share all indexing code.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dn {

typedef __bf16 bf16;
typedef bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16;
typedef float f32x4 __attribute__((ext_vector_type(4)));

enum : int { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2, DT_I32 = 3, DT_I64 = 4 };

constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

__device__ __forceinline__ int pi_k(int q, int e) { return (e < 4) ? (4 * q + e) : (12 + 4 * q + e); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------------------
// scalar loads with a run-time element type (gates, segment ids)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float ld_f(const void* p, int64_t i, int dt) {
  if (dt == DT_BF16) return (float)((const bf16*)p)[i];
  if (dt == DT_F16) return (float)((const f16*)p)[i];
  return ((const float*)p)[i];
}

__device__ __forceinline__ int64_t ld_i(const void* p, int64_t i, int dt) {
  if (dt == DT_I64) return ((const int64_t*)p)[i];
  return (int64_t)((const int32_t*)p)[i];
}

template <class T> __device__ __forceinline__ float to_f(T x) { return (float)x; }

template <class T> __device__ __forceinline__ T from_f(float x);
template <> __device__ __forceinline__ float from_f<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16 from_f<bf16>(float x) { return (bf16)x; }
template <> __device__ __forceinline__ f16 from_f<f16>(float x) { return (f16)x; }

// round a float through T and back (models storing into a T tensor)
template <class T> __device__ __forceinline__ float round_as(float x) { return (float)from_f<T>(x); }

// 4 contiguous elements -> floats
template <class T> __device__ __forceinline__ void ld4(const T* p, float* o) {
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = to_f(p[i]);
}
template <> __device__ __forceinline__ void ld4<float>(const float* p, float* o) {
  float4 x = *reinterpret_cast<const float4*>(p);
  o[0] = x.x; o[1] = x.y; o[2] = x.z; o[3] = x.w;
}
template <> __device__ __forceinline__ void ld4<bf16>(const bf16* p, float* o) {
  bf16x4 x = *reinterpret_cast<const bf16x4*>(p);
  o[0] = (float)x[0]; o[1] = (float)x[1]; o[2] = (float)x[2]; o[3] = (float)x[3];
}

// The 8 fragment-order elements of a row slab (rowp[4q..4q+3], rowp[16+4q..])
// held exactly as loaded, so the loads can be issued long before the values
// are needed (the wait lands at the first use, not at the load).
template <class T> struct Raw8 {
  typedef T V __attribute__((ext_vector_type(4)));
  V a, b;
  __device__ __forceinline__ void load(const T* rowp, int q) {
    a = *reinterpret_cast<const V*>(rowp + 4 * q);
    b = *reinterpret_cast<const V*>(rowp + 16 + 4 * q);
  }
  __device__ __forceinline__ void to(float* x) const {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = (float)a[e];
      x[4 + e] = (float)b[e];
    }
  }
};

template <class T> __device__ __forceinline__ void st4(T* p, const float* v) {
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = from_f<T>(v[i]);
}
template <> __device__ __forceinline__ void st4<float>(float* p, const float* v) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}
template <> __device__ __forceinline__ void st4<bf16>(bf16* p, const float* v) {
  bf16x4 x;
  x[0] = (bf16)v[0]; x[1] = (bf16)v[1]; x[2] = (bf16)v[2]; x[3] = (bf16)v[3];
  *reinterpret_cast<bf16x4*>(p) = x;
}

// ---------------------------------------------------------------------------
// MFMA fragments
// ---------------------------------------------------------------------------
template <bool BF> struct Frag;
template <> struct Frag<true> { bf16x8 v; };
template <> struct Frag<false> { float v[8]; };

template <bool BF> __device__ __forceinline__ Frag<BF> make_frag(const float* x);
template <> __device__ __forceinline__ Frag<true> make_frag<true>(const float* x) {
  Frag<true> f;
#pragma unroll
  for (int e = 0; e < 8; ++e) f.v[e] = (bf16)x[e];
  return f;
}
template <> __device__ __forceinline__ Frag<false> make_frag<false>(const float* x) {
  Frag<false> f;
#pragma unroll
  for (int e = 0; e < 8; ++e) f.v[e] = x[e];
  return f;
}

__device__ __forceinline__ void mma(f32x4& acc, const Frag<true>& a, const Frag<true>& b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.v, b.v, acc, 0, 0, 0);
}
__device__ __forceinline__ void mma(f32x4& acc, const Frag<false>& a, const Frag<false>& b) {
#pragma unroll
  for (int e = 0; e < 8; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.v[e], b.v[e], acc, 0, 0, 0);
}

// Fragment from a row-major row pointer at the slab start (k0 already added):
// elements rowp[4q..4q+3] and rowp[16+4q..16+4q+3].
template <bool BF, class T> __device__ __forceinline__ Frag<BF> frag_row(const T* rowp, int q) {
  float x[8];
  ld4<T>(rowp + 4 * q, x);
  ld4<T>(rowp + 16 + 4 * q, x + 4);
  return make_frag<BF>(x);
}

// Fragment from a column of row-major storage: elements colp[pi(q,e) * stride].
template <bool BF, class T>
__device__ __forceinline__ Frag<BF> frag_col(const T* colp, int64_t stride, int q) {
  float x[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = to_f(colp[(int64_t)pi_k(q, e) * stride]);
  return make_frag<BF>(x);
}

// Two stacked accumulator tiles (rows 0-15 and 16-31 of a slab) as a fragment.
template <bool BF> __device__ __forceinline__ Frag<BF> frag_from_acc(const f32x4& c0, const f32x4& c1) {
  float x[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
  return make_frag<BF>(x);
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// Workgroup barrier that orders LDS only: waits for this wave's LDS
// operations, not for its outstanding global loads, so prefetches issued
// before the barrier stay in flight across it.  (__syncthreads() also drains
// the vector-memory counter.)  Not for exchanging data through global memory.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// ---------------------------------------------------------------------------
// Precision policy.  "bf16" mode runs plain products on bf16 MFMA and the
// products that set the output accuracy as split-bf16 products: an fp32
// operand x is carried as hi = bf16(x), lo = bf16(x - hi) (16 significant
// bits) and a*b ~ a_hi*b_hi + a_hi*b_lo + a_lo*b_hi, all accumulated in fp32.
// "fp32" mode runs every product on v_mfma_f32_16x16x4_f32.
// ---------------------------------------------------------------------------
template <bool BF> struct Pol;

template <> struct Pol<true> {
  using F1 = Frag<true>;
  struct F3 { Frag<true> hi, lo; };
  static __device__ __forceinline__ F1 f1(const float* x) { return make_frag<true>(x); }
  static __device__ __forceinline__ F3 f3(const float* x) {
    F3 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const bf16 h = (bf16)x[e];
      r.hi.v[e] = h;
      r.lo.v[e] = (bf16)(x[e] - (float)h);
    }
    return r;
  }
  static __device__ __forceinline__ F1 hi(const F3& a) { return a.hi; }
  static __device__ __forceinline__ void m11(f32x4& c, const F1& a, const F1& b) { mma(c, a, b); }
  static __device__ __forceinline__ void m13(f32x4& c, const F1& a, const F3& b) { mma(c, a, b.hi); mma(c, a, b.lo); }
  static __device__ __forceinline__ void m33(f32x4& c, const F3& a, const F3& b) {
    mma(c, a.hi, b.hi);
    mma(c, a.hi, b.lo);
    mma(c, a.lo, b.hi);
  }
};

template <> struct Pol<false> {
  using F1 = Frag<false>;
  using F3 = Frag<false>;
  static __device__ __forceinline__ F1 f1(const float* x) { return make_frag<false>(x); }
  static __device__ __forceinline__ F3 f3(const float* x) { return make_frag<false>(x); }
  static __device__ __forceinline__ F1 hi(const F3& a) { return a; }
  static __device__ __forceinline__ void m11(f32x4& c, const F1& a, const F1& b) { mma(c, a, b); }
  static __device__ __forceinline__ void m13(f32x4& c, const F1& a, const F3& b) { mma(c, a, b); }
  static __device__ __forceinline__ void m33(f32x4& c, const F3& a, const F3& b) { mma(c, a, b); }
};

// ---------------------------------------------------------------------------
// Operand storage.  Intermediates are written in the lane order of the MFMA
// operand that consumes them ("fragment-native"): a 16 x 32 operand slab is 64
// lanes x 8 elements, lane (r, q) holding row r and reduction indices
// pi(q, 0..7), so a consumer loads 16 (bf16) or 32 (fp32) contiguous bytes per
// lane.  An accumulator tile of the transposed product (lane (c, q) holding
// rows 4q..4q+3 of column c) is one half (e = 0..3 or 4..7) of such a slab.
// Operands of split products are stored split (bf16 mode: hi and lo bf16
// arrays; fp32 mode: one fp32 array, lo aliases hi).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int fofs(int tile, int slab, int lane) { return ((tile * 4 + slab) * 64 + lane) * 8; }
__device__ __forceinline__ int cofs(int rtile, int ctile, int nct, int lane) { return ((rtile * nct + ctile) * 64 + lane) * 4; }

template <bool BF> struct Store;

template <> struct Store<true> {
  using ST = bf16;
  using F1 = Pol<true>::F1;
  using F3 = Pol<true>::F3;
  static __device__ __forceinline__ F1 fa(const bf16* p) {
    F1 f;
    f.v = *reinterpret_cast<const bf16x8*>(p);
    return f;
  }
  static __device__ __forceinline__ F3 fa3(const bf16* hi, const bf16* lo) {
    F3 r;
    r.hi = fa(hi);
    r.lo = fa(lo);
    return r;
  }
  static __device__ __forceinline__ void st8(bf16* p, const float* x) {
    bf16x8 h;
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = (bf16)x[e];
    *reinterpret_cast<bf16x8*>(p) = h;
  }
  static __device__ __forceinline__ void st8s(bf16* hi, bf16* lo, const float* x) {
    bf16x8 h, l;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      h[e] = (bf16)x[e];
      l[e] = (bf16)(x[e] - (float)h[e]);
    }
    *reinterpret_cast<bf16x8*>(hi) = h;
    *reinterpret_cast<bf16x8*>(lo) = l;
  }
  static __device__ __forceinline__ void stf(bf16* p, const F1& f) { *reinterpret_cast<bf16x8*>(p) = f.v; }
  static __device__ __forceinline__ void st4(bf16* p, const float* x) {
    bf16x4 h;
#pragma unroll
    for (int e = 0; e < 4; ++e) h[e] = (bf16)x[e];
    *reinterpret_cast<bf16x4*>(p) = h;
  }
  static __device__ __forceinline__ void st4s(bf16* hi, bf16* lo, const float* x) {
    bf16x4 h, l;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      h[e] = (bf16)x[e];
      l[e] = (bf16)(x[e] - (float)h[e]);
    }
    *reinterpret_cast<bf16x4*>(hi) = h;
    *reinterpret_cast<bf16x4*>(lo) = l;
  }
  // fragment (pi order) from a row-major row pointer at the slab start
  static __device__ __forceinline__ F1 f1(const bf16* rowp, int q) {
    const bf16x4 a = *reinterpret_cast<const bf16x4*>(rowp + 4 * q);
    const bf16x4 b = *reinterpret_cast<const bf16x4*>(rowp + 16 + 4 * q);
    F1 f;
    f.v = bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    return f;
  }
  static __device__ __forceinline__ F3 f3(const bf16* hi, const bf16* lo, int q) {
    F3 r;
    r.hi = f1(hi, q);
    r.lo = f1(lo, q);
    return r;
  }
  static __device__ __forceinline__ void put(bf16* hi, bf16* lo, int i, float v) {
    const bf16 h = (bf16)v;
    hi[i] = h;
    lo[i] = (bf16)(v - (float)h);
  }
};

template <> struct Store<false> {
  using ST = float;
  using F1 = Pol<false>::F1;
  using F3 = Pol<false>::F3;
  static __device__ __forceinline__ F1 fa(const float* p) {
    F1 f;
    const f32x4 a = *reinterpret_cast<const f32x4*>(p);
    const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) { f.v[e] = a[e]; f.v[4 + e] = b[e]; }
    return f;
  }
  static __device__ __forceinline__ F3 fa3(const float* hi, const float*) { return fa(hi); }
  static __device__ __forceinline__ void st8(float* p, const float* x) {
    *reinterpret_cast<f32x4*>(p) = f32x4{x[0], x[1], x[2], x[3]};
    *reinterpret_cast<f32x4*>(p + 4) = f32x4{x[4], x[5], x[6], x[7]};
  }
  static __device__ __forceinline__ void st8s(float* hi, float*, const float* x) { st8(hi, x); }
  static __device__ __forceinline__ void stf(float* p, const F1& f) { st8(p, f.v); }
  static __device__ __forceinline__ void st4(float* p, const float* x) {
    *reinterpret_cast<f32x4*>(p) = f32x4{x[0], x[1], x[2], x[3]};
  }
  static __device__ __forceinline__ void st4s(float* hi, float*, const float* x) { st4(hi, x); }
  static __device__ __forceinline__ F1 f1(const float* rowp, int q) { return frag_row<false, float>(rowp, q); }
  static __device__ __forceinline__ F3 f3(const float* hi, const float*, int q) { return f1(hi, q); }
  static __device__ __forceinline__ void put(float* hi, float*, int i, float v) { hi[i] = v; }
};

// B fragments of the two halves of a 32 x 32 identity: A (16 x 32) times
// ident(0) / ident(1) is the left / right 16 x 16 half of A, delivered in
// accumulator layout, i.e. transposed relative to the A fragment (exact: one
// product by 1 per output element).
template <bool BF> __device__ __forceinline__ Frag<BF> ident_frag(int half, int r16, int q) {
  float x[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = (pi_k(q, e) == 16 * half + r16) ? 1.f : 0.f;
  return make_frag<BF>(x);
}

// XCD-aware block index.  Consecutive workgroups of a launch are dealt to the
// 8 XCDs round-robin; this remaps the linear block id so that each XCD works
// on one contiguous range of the logical grid (x fastest), keeping the
// operands those blocks share in one XCD's L2.  Identity when the grid does
// not divide evenly.
__device__ __forceinline__ void xcd_block(int& x, int& y, int& z) {
  const int gx = gridDim.x, gy = gridDim.y;
  const int tot = gx * gy * gridDim.z;
  int id = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
  if ((tot & 7) == 0) id = (id & 7) * (tot >> 3) + (id >> 3);
  x = id % gx;
  id /= gx;
  y = id % gy;
  z = id / gy;
}

// 8 fragment values (pi order) from a row-major row pointer at the slab start
template <class T> __device__ __forceinline__ void row8(const T* rowp, int q, float* x) {
  ld4<T>(rowp + 4 * q, x);
  ld4<T>(rowp + 16 + 4 * q, x + 4);
}

}  // namespace dn
