/*
 * deltanet_amd.h -- C ABI of the MI355X (gfx950) delta-rule recurrence core.
 *
 * Drop-in boundary for the forward path of maelie-labs/deltanet-tpu v0.3.0.
 * In the reference the two device boundaries of chunk_gdn2 are Pallas calls
 * inside a jax.custom_vjp (src/deltanet_tpu/gdn2.py:1262-1276 prepass,
 * 1331-1347 sequential state/output pass, both launched by
 * _chunked_recurrence_fwd gdn2.py:1176-1389) and the decode step is one XLA
 * fusion (gdn2.py:2471-2478).  Each entry point below is what an XLA-FFI
 * custom call (jax.ffi.ffi_call) or a ctypes / torch host binding would bind
 * in their place.  Everything is plain C: device pointers, sizes, flags and an
 * opaque HIP stream.  The library never allocates device memory for a call:
 * scratch comes in through the `workspace` argument, whose size the caller
 * asks for first.
 *
 * Tensor layouts (all row-major / C-contiguous, element strides implied):
 *   q, k   (B, L, Hk, K)         v, out (B, L, Hv, V)
 *   g, b   (B, L, Hx, Cx)        w      (B, L, Hx, Cx)    (prefill: float32)
 *          Hx in {1, Hk, Hv}; Cx in {1, K} for g/b and {1, V} for w.
 *          A gate with Hx == Hk is shared by the G = Hv/Hk value heads of a
 *          key head (value head hv reads head hv / G); Hx == 1 is shared by
 *          all heads; Cx == 1 is one scalar per head.
 *   seg    (B, L) or (L,) int32 / int64 segment (document) ids, or NULL.
 *   state  (B, Hv, K, V) float32 (prefill) / float32 or bfloat16 (decode).
 *
 * Return value of every call: 0 on success, a negative DN_E* code otherwise;
 * dn_last_error() gives the message of the calling thread's last failure.
 */
#ifndef DELTANET_AMD_H_
#define DELTANET_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DN_ABI_VERSION 2

/* element types */
enum { DN_F32 = 0, DN_BF16 = 1, DN_F16 = 2, DN_I32 = 3, DN_I64 = 4 };

/* error codes */
enum {
  DN_OK = 0,
  DN_E_INVALID = -1,   /* bad shape / dtype / flag combination            */
  DN_E_WORKSPACE = -2, /* workspace missing or smaller than required      */
  DN_E_LAUNCH = -3,    /* HIP launch / runtime error                      */
  DN_E_ABI = -4        /* args struct built against another ABI version   */
};

/* Arguments of one chunked prefill call (chunk_gdn2 forward, is_inference).
 * Mirrors the static flags and operands of the reference's inference op
 * (_get_inference_custom_vjp, gdn2.py:1392-1443) plus the wrapper-level
 * semantics it performs before launching (gdn2.py:1970-2125), which this
 * library applies inside its kernels instead of as extra HBM passes. */
typedef struct dn_prefill_args {
  int32_t abi_version;          /* must be DN_ABI_VERSION                      */
  int32_t B, L, Hk, Hv, K, V;   /* tensor dims; K == V == 128 (gdn2.py:1897)   */
  int32_t t0, nt;               /* token range [t0, t0+nt) of this call; t0 is a
                                   multiple of 128 (streaming prefill block)   */
  const void* q;                /* (B,L,Hk,K)                                   */
  const void* k;                /* (B,L,Hk,K)                                   */
  const void* v;                /* (B,L,Hv,V)                                   */
  int32_t qk_dtype, v_dtype;    /* q/k: DN_F32 / DN_BF16 / DN_F16; v: F32 / BF16 */
  const void* g; int32_t g_dtype, g_heads, g_chans;   /* gates: DN_F32          */
  const void* b; int32_t b_dtype, b_heads, b_chans;
  const void* w; int32_t w_dtype, w_heads, w_chans;
  const void* seg;              /* NULL or segment ids                          */
  int32_t seg_dtype;            /* DN_I32 / DN_I64                              */
  int32_t seg_batched;          /* 1: seg is (B,L); 0: seg is (L,) shared       */
  const float* init_state;      /* NULL or (B,Hv,K,V) f32; may alias final_state */
  const int32_t* init_seg;      /* NULL or (B,) initial_state_segment_id         */
  void* out;                    /* (B,L,Hv,V) of v_dtype                         */
  float* final_state;           /* NULL or (B,Hv,K,V) f32                        */
  float scale;                  /* query scale (1/sqrt(K) by default)            */
  int32_t qk_l2norm;            /* L2-normalise q and k                          */
  int32_t fuse_prologue;        /* raw g/b/w: g=-exp(min(g,5)), b,w=sigmoid      */
  int32_t stability_guard;      /* clamps b>=0, g<=-1e-6 (not the state cap)     */
  int32_t precision;            /* 0 = "bf16", 1 = "fp32"                        */
  int32_t gates_at_hv;          /* 1: execute per value head (g or b has Hv heads) */
  int32_t block_tokens;         /* internal token block (multiple of 128), 0=auto */
  int32_t recompute_states;     /* training backward (dn_prefill_bwd_raw): keep only
                                   token-block boundary states and recompute the
                                   per-chunk states block by block, as
                                   recompute_states=True (gdn2.py:1614-1630); the
                                   gradients are bit-identical, the workspace smaller */
} dn_prefill_args;

/* Bytes of device workspace dn_prefill_fwd needs for these arguments. */
size_t dn_prefill_workspace_size(const dn_prefill_args* a);

/* Chunked WY prefill: replaces the prepass + sequential state pallas_calls of
 * _chunked_recurrence_fwd (gdn2.py:1262-1276, 1331-1347) and the wrapper work
 * around them (gate broadcast, segment canonicalisation, padding, q/k L2-norm,
 * value-head fusion; gdn2.py:1970-2125, 2198-2238).  Enqueues on `stream`
 * (a hipStream_t; NULL = default stream); never synchronises. */
int dn_prefill_fwd(const dn_prefill_args* a, void* workspace, size_t workspace_bytes, void* stream);

/* Allocation-free prefill (no counterpart in the reference: for callers that
 * cannot allocate device memory -- code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments, results and
 * errors as dn_prefill_fwd, but the scratch is a file-scope device array of
 * DN_NOALLOC_SCRATCH_BYTES that each GPU holds from the library's first use on
 * it until the process ends; the call allocates nothing.  The token range is
 * processed in blocks small enough for that scratch (bit-identical results);
 * a shape whose single 128-token block of every (batch, head) does not fit is
 * rejected with DN_E_WORKSPACE.  Every call on a GPU shares that GPU's array:
 * calls that overlap on one GPU (two streams, two threads) race, so the
 * caller serialises them (one stream, or events between streams). */
#define DN_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int dn_prefill_fwd_noalloc(const dn_prefill_args* a, void* stream);

/* Arguments of one single-token decode step (gdn2_decode_step, gdn2.py:2289-2490). */
typedef struct dn_decode_args {
  int32_t abi_version;
  int32_t B, Hk, Hv, K, V;      /* K == V == 128                                 */
  const void* q;                /* (B,Hk,K)                                      */
  const void* k;                /* (B,Hk,K)                                      */
  const void* v;                /* (B,Hv,V)                                      */
  int32_t qk_dtype, v_dtype;
  const void* g; int32_t g_dtype, g_heads, g_chans;   /* (B,Hx,Cx) */
  const void* b; int32_t b_dtype, b_heads, b_chans;
  const void* w; int32_t w_dtype, w_heads, w_chans;
  const void* state_in;  int32_t state_in_dtype;      /* (B,Hv,K,V) f32 / bf16  */
  void* state_out;       int32_t state_out_dtype;     /* may alias state_in      */
  const uint8_t* reset;         /* NULL or (B,) : clear the state first          */
  void* out;                    /* (B,Hv,V) of v_dtype                            */
  float scale;
  int32_t qk_l2norm;
  int32_t stability_guard;      /* clamps + Frobenius cap of the new state        */
  float stability_tau;
} dn_decode_args;

/* Decode step: replaces the XLA fusion of gdn2.py:2393-2489 (upcast, clamp,
 * reset, GQA repeat, L2-norm, decay/erase/write/readout, cap, state cast). */
int dn_decode_step(const dn_decode_args* a, void* stream);

/* T consecutive decode steps in one launch (no counterpart in the reference:
 * the multi-token decode it lists as a next step, for speculative decoding and
 * small-batch serving, where one state read and write per T tokens replaces T).
 * Same arguments as dn_decode_step except that every per-token tensor carries
 * a token axis after the batch axis: q, k (B,T,Hk,K); v, out (B,T,Hv,V); gates
 * (B,T,Hx,Cx); reset NULL or (B,T), clearing the state before that token.  The
 * result is the recurrence of T chained dn_decode_step calls; stability_guard
 * caps after every token.  T >= 6 without the guard runs as 16-token chunks in
 * the chunked WY form (fp32 products on the fp32 matrix cores when either state
 * is fp32, split bf16 for a bf16 state) and carries the state in fp32 across
 * the T tokens, converting it to state_out_dtype once; the other launches
 * round a bf16 state after every token, as chained steps do.  A bf16 state
 * therefore agrees with chained steps to bf16 rounding.  T == 1 is
 * dn_decode_step. */
int dn_decode_steps(const dn_decode_args* a, int32_t T, void* stream);

/* Arguments of the training backward of the chunked recurrence.  All tensors
 * are float32 and already prepared by the caller: q (scaled, normalised), k,
 * g (clamped, natural-log decay) and b at H value heads with K channels each;
 * v and w at H heads with V channels.  The wrapper's elementwise steps
 * (prologue, L2-norm, gate broadcast, GQA repeat) are differentiated by the
 * caller, which sums the returned gradients back to its own layouts. */
typedef struct dn_backward_args {
  int32_t abi_version;
  int32_t B, L, H, K, V;        /* K == V == 128                                 */
  const void* q;                /* (B,L,H,K) f32                                 */
  const void* k;                /* (B,L,H,K) f32                                 */
  const void* v;                /* (B,L,H,V) f32                                 */
  const void* g;                /* (B,L,H,K) f32, <= 0                           */
  const void* b;                /* (B,L,H,K) f32                                 */
  const void* w;                /* (B,L,H,V) f32                                 */
  const int32_t* seg;           /* NULL or (B,L) canonical segment ids: nondecreasing,
                                   the initial state belongs to id 0              */
  const void* init_state;       /* NULL or (B,H,K,V) f32                         */
  const void* d_out;            /* (B,L,H,V) f32 cotangent of the output          */
  const void* d_final;          /* NULL or (B,H,K,V) f32 cotangent of the final state */
  void *dq, *dk, *dv, *dg, *db, *dw;  /* f32, shapes of q k v g b w            */
  void* d_init;                 /* NULL or (B,H,K,V) f32 (needs init_state)       */
  int32_t recompute_states;     /* 0: one pass over the whole sequence, every chunk's
                                   state in the workspace.  1: token blocks, the
                                   workspace holding one block's chunk products plus
                                   the state at each block boundary; a forward pass
                                   stores those states, then the blocks run from the
                                   last to the first, each recomputing its chunk
                                   states from the boundary state before it (the
                                   reference's _recompute_chunk_states_kernel,
                                   gdn2.py:655-695).  Bit-identical gradients. */
} dn_backward_args;

/* Workspace bytes dn_prefill_bwd needs (0 if the arguments are invalid):
 * about 545 KB per (batch, head, 64-token chunk); with recompute_states, 545 KB
 * per (batch, head, chunk of one token block) plus 64 KB per (batch, head) for
 * each token block when there is more than one: the states entering the
 * interior blocks, and the state gradient carried from one block to the one
 * before it.  The block is the smallest whole number of chunks giving at least
 * 1024 (batch, head, chunk) units per launch. */
size_t dn_prefill_bwd_workspace_size(const dn_backward_args* a);

/* Backward of the chunked recurrence: replaces the reference's custom-VJP
 * backward (gdn2.py:1446-1769: reverse state scan gdn2.py:698-769 and the
 * analytical prepass adjoint gdn2.py:243-493, 496-582).  Gradients of
 * sum(out * d_out) + sum(final * d_final) are written (not accumulated). */
int dn_prefill_bwd(const dn_backward_args* a, void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes dn_prefill_bwd_raw needs (0 if the arguments are invalid):
 * dn_prefill_bwd_workspace_size at H = Hv (with a->recompute_states) plus the
 * prepared inputs and their gradients as f32 arrays: seven (B,L,Hv,128), two
 * (B,L,Hk,128) (q, k) and two for g and b, (B,L,Hk,128) when both have Hk
 * heads and (B,L,Hv,128) otherwise. */
size_t dn_prefill_bwd_raw_workspace_size(const dn_prefill_args* a);

/* Backward of the whole training op from the forward's own arguments: the
 * custom VJP of gdn2.py:1446-1769 together with the wrapper steps it sits
 * behind (gdn2.py:1970-2125: nonpositive clamp with its pass-through gradient,
 * guard clamps, fused prologue, q/k L2-norm and scale with the cast back to the
 * input dtype, gate broadcast, GQA head mapping, segment canonicalisation).
 * `a` is the dn_prefill_fwd argument block of the forward call (t0 = 0,
 * nt = L; out / final_state are not read).  d_out (B,L,Hv,V) in the output's
 * element type (v_dtype), d_final NULL or (B,Hv,K,V) f32.  Gradients are written
 * in the raw layouts, like the reference's VJP in the input dtypes: dq, dk
 * (B,L,Hk,K) in qk_dtype and dv (B,L,Hv,V) in v_dtype (f32 results rounded to
 * nearest even); dg, db, dw (B,L,H,C) of their gate and d_init NULL or
 * (B,Hv,K,V) in f32.  Every tensor must be dense row-major in the layout and
 * element type the header gives (strides are implied, never passed): a
 * channel-wise write gate at Hv heads with neither fuse_prologue nor
 * stability_guard is read in place by the recurrence kernels, every other
 * gate layout is first staged into the workspace; without fuse_prologue such
 * a gate's dw is written in place by the recurrence kernels too.  a->precision
 * selects the arithmetic as in the forward: "bf16" (0) runs the state scans and
 * the chunk gradient products as split-bf16 MFMA products (hi + lo words,
 * fp32 accumulation), "fp32" (1) runs every product in fp32. */
int dn_prefill_bwd_raw(const dn_prefill_args* a, const void* d_out, const void* d_final,
                       void* dq, void* dk, void* dv, void* dg, void* db, void* dw, void* d_init,
                       void* workspace, size_t workspace_bytes, void* stream);

/* In-place Frobenius cap S <- S * min(1, tau / sqrt(||S||_F^2 + 1e-6)) of
 * `nmat` consecutive (rows x cols) float32 matrices (the stability_guard cap of
 * gdn2.py:2180-2188 / 2224-2226 / 2236-2238). */
int dn_state_frob_cap(float* state, int64_t nmat, int32_t rows, int32_t cols, float tau, void* stream);

/* Kernel timing instrumentation (no counterpart in the reference; for
 * benchmarks and profilers).  Between dn_profile_begin() and dn_profile_end()
 * every dn_prefill_fwd call (from any thread of the process) records HIP events on its
 * stream around each of its kernels (prepass, chain; kind 1 is no longer
 * recorded: the value products run inside the prepass) and every
 * dn_decode_step / dn_decode_steps call around its kernel, and every
 * dn_prefill_bwd call around its four kernels together.  dn_profile_end() waits for those
 * events and writes, per kernel kind, the summed duration in milliseconds
 * and the number of launches (arrays of DN_PROFILE_KINDS entries). */
#define DN_PROFILE_KINDS 5   /* 0 prepass, 1 (unused), 2 chain, 3 decode, 4 backward */
int dn_profile_begin(void);
int dn_profile_end(double* ms_sum, int64_t* launches);

/* Message of the calling thread's last failed call ("" if none). */
const char* dn_last_error(void);

/* DN_ABI_VERSION the library was built with. */
int dn_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif /* DELTANET_AMD_H_ */
