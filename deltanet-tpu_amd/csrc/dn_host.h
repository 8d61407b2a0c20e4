// Host-side declarations shared by the kernel translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "deltanet_amd.h"

namespace dn {

// Kernel parameter block of one prefill token block (passed by value).
struct PF {
  int B, L, Hk, Hv, G;       // tensor dims, G = Hv / Hk
  int Hx, Vp, gates_at_hv;   // execution heads, value width per execution head
  int t0, nt, NCb;           // token block [t0, t0+nt), chunks in the block
  int ncg;                   // 256-column groups of the value width (k_output)
  const void *q, *k, *v;
  int v_dt;
  const void* g; int g_dt, g_h, g_c;
  const void* b; int b_dt, b_h, b_c;
  const void* w; int w_dt, w_h, w_c;
  const void* seg; int seg_dt, seg_batched;
  const float* init; int has_init;
  const int32_t* init_seg;
  void* out;
  float* fin;
  float scale; int l2norm, fuse, guard;
  // workspace arrays (one unit = one (batch, exec head, chunk))
  int32_t* flags;            // [B][NCb][2] : is_new_doc, all_same_doc
  float* dvec;               // [unit][K]    : e^{Lambda_end}
  void* Pn;                  // [unit][K][K] : -ke^T W (bf16 in bf16 mode)
  float* Q;                  // [unit][K][Vp]: ke^T U
  float* X;                  // [unit][C][K] : qe - M W   (effective queries)
  float* Oi;                 // [unit][C][Vp]: M U        (intra-chunk output)
  float* St;                 // [unit][Vp][K]: entry state of the chunk, transposed
  float *beT, *keT, *Mg, *qe;  // prepass scratch: [K][C], [K][C], [C][C], [C][K]
};

// Records the message for dn_last_error() and returns `code`.
int set_error(int code, const char* msg);

// Kernel timing (dn_profile_begin / dn_profile_end): returns true when the
// calling thread is profiling; mark() records an event for `kind` on `st`
// (call it once before and once after each launch).
bool profiling();
void prof_mark(int kind, hipStream_t st, bool after);

}  // namespace dn
