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
  int nct;                   // 16-column tiles of the value width (Vp / 16)
  // Workspace, per unit = (batch, exec head, chunk).  Every operand array is
  // fragment-native for its consumer (F = [tile][slab][lane][8] elements of a
  // 16 x 32 MFMA operand slab, C = [row tile][col tile][lane][4] accumulator
  // tiles).  Split operands have a high and a low array (bf16 mode; in fp32
  // mode the low pointer aliases the high one).  "ST" = bf16 in bf16 mode,
  // fp32 in fp32 mode.
  void* PnA;                 // F  [8][4]      ST : Pn = -ke^T W, rows = state row (chain A)
  float* QC;                 // C  [8][nct]    f32: Q = ke^T U (chain accumulator init)
  void *XAh, *XAl;           // F  [8][4]      ST : X = qe - M W, rows = token (chain output B)
  float* OiT;                // C  [8][nct]    f32: (M U)^T tiles (chain output accumulator init)
  void* BeB;                 // F  [8][4]      ST : (b k e^Lambda)^T, first document
  void *KeBh, *KeBl;         // F  [8][4]      ST : (k e^{Lend - Lambda})^T, last document
  void *MAh, *MAl;           // F  [8][4]      ST : M, rows = token
  float* QeA;                // F  [8][4]      f32: q e^Lambda, first document
  void* sink;                // 1 KB the chain's output lanes past the last token store into
};

// Records the message for dn_last_error() and returns `code`.
int set_error(int code, const char* msg);

// Kernel timing (dn_profile_begin / dn_profile_end): returns true when the
// calling thread is profiling; mark() records an event for `kind` on `st`
// (call it once before and once after each launch).
bool profiling();
void prof_mark(int kind, hipStream_t st, bool after);

}  // namespace dn
