/*
 * ssa_mi355x.h -- C ABI of the MI355X (gfx950) SSA flash-attention library
 * (libssa_mi355x.so).
 *
 * SSA = softmax-substituted attention: logits s = scale * q.k are replaced by
 * t(s) = n * sign(s) * ln(1 + b |s|) before a row softmax.  This library is the
 * device half of the drop-in replacement for the reference's Triton launch
 * layer; the Python host side (luciole-1b_amd/SSA) binds these entry points
 * with ctypes.
 *
 * Conventions
 *  - Every entry point validates its arguments on the host and returns a
 *    status (SSA_OK = 0) before any launch; nothing is launched on error.
 *  - The library never allocates or frees device memory.  Outputs and
 *    workspaces are passed in by the caller (ssa_bwd_noalloc instead uses a
 *    fixed-size static device array of the library's code object).
 *  - Work is enqueued asynchronously on `stream` (a hipStream_t; NULL = the
 *    default stream).  No entry point synchronises the device or reads device
 *    memory on the host (n and b are read by the kernels through pointers).
 *  - Tensors are [batch, heads, seqlen, head_dim] views described by a base
 *    pointer and element strides for the first three dimensions; the last
 *    (head_dim) stride must be 1.  Base pointers must be 16-byte aligned, the
 *    three strides non-negative multiples of 8 elements, and the row
 *    (seqlen) stride below 2^24 elements.
 *  - Results are bitwise deterministic run to run: no floating-point atomics,
 *    fixed-order reductions only.
 */
#ifndef SSA_MI355X_H
#define SSA_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SSA_ABI_VERSION 6

/* Status codes. */
enum {
  SSA_OK = 0,
  SSA_ERR_NULL_POINTER = 1,   /* a required pointer is NULL                       */
  SSA_ERR_SHAPE = 2,          /* bad batch/heads/seqlen (e.g. Hq % Hkv != 0), or  */
                              /* beyond the int32 launch limits: seqlen <= 2^30,  */
                              /* B * Hq * ceil(seqlen / 128) <= 2^28, and query   */
                              /* rows B * Hq * seqlen (packed: Hq * total_tokens) */
                              /* <= INT32_MAX; decode: capacity <= 2^30          */
  SSA_ERR_HEAD_DIM = 3,       /* head_dim not one of 32, 64, 128, 256 (fp32: 16)  */
  SSA_ERR_DTYPE = 4,          /* dtype not an SSA_DTYPE_* (decode: bf16 / fp16)   */
  SSA_ERR_ALIGNMENT = 5,      /* layout: base pointer not 16-byte aligned, a      */
                              /* stride negative or not a multiple of 8, or the   */
                              /* row stride >= 2^24 elements                      */
  SSA_ERR_LAUNCH = 6,         /* the HIP runtime rejected a kernel launch         */
  SSA_ERR_CU_SEQLENS = 7,     /* varlen: bad document table                       */
  SSA_ERR_SCRATCH = 8         /* ssa_bwd_noalloc: the problem's Delta + partials  */
                              /* exceed SSA_NOALLOC_SCRATCH_BYTES                 */
};

/*
 * Element types of q/k/v/out/dout/dq/dk/dv.  bf16 / fp16 run on the MFMA
 * kernels at head dims 32, 64, 128.  fp32 -- the reference's fp32-operand
 * path (training/train/train_ssa_triton/SSA/ssa_triton_kernel.py:766-772,
 * 819-825) -- runs on fp32 vector-ALU kernels (head dims 16, 32, 64, 128,
 * 256) that keep every product in fp32: full precision, a fraction of the
 * bf16 throughput.  bf16 / fp16 at head dim 256 (the reference takes every
 * power-of-two head dim, ssa_triton_kernel.py:761-764) run on the same
 * vector-ALU kernels, elements widened to fp32 on load.  On the vector-ALU
 * kernels the dS' workspace is not used (dq recomputes the scores); the
 * decode step takes bf16 / fp16 at head dims 32, 64, 128.
 */
enum { SSA_DTYPE_BF16 = 0, SSA_DTYPE_FP16 = 1, SSA_DTYPE_FP32 = 2 };

/* A [B, H, S, D] tensor view; strides in elements, stride(D) == 1. */
typedef struct ssa_tensor4 {
  void* ptr;
  int64_t stride_b;
  int64_t stride_h;
  int64_t stride_s;
} ssa_tensor4;

typedef struct ssa_fwd_args {
  ssa_tensor4 q;        /* [B, Hq,  N, D] */
  ssa_tensor4 k;        /* [B, Hkv, N, D] */
  ssa_tensor4 v;        /* [B, Hkv, N, D] */
  ssa_tensor4 out;      /* [B, Hq,  N, D], written */
  float* m;             /* [B, Hq, N] contiguous fp32, written: log2(sum_j exp(t_ij)) */
  const float* ssa_n;   /* device fp32 scalar n */
  const float* ssa_b;   /* device fp32 scalar b */
  int32_t batch, heads_q, heads_kv, seqlen, head_dim;
  int32_t dtype;        /* SSA_DTYPE_* */
  int32_t causal;       /* 0 / 1: top-left aligned causal mask */
  float softmax_scale;
} ssa_fwd_args;

typedef struct ssa_bwd_args {
  ssa_tensor4 q, k, v;  /* as in ssa_fwd_args */
  ssa_tensor4 out;      /* forward output */
  ssa_tensor4 dout;     /* incoming gradient, [B, Hq, N, D] */
  ssa_tensor4 dq;       /* written, [B, Hq,  N, D] */
  ssa_tensor4 dk;       /* written, [B, Hkv, N, D] */
  ssa_tensor4 dv;       /* written, [B, Hkv, N, D] */
  const float* m;       /* [B, Hq, N] fp32 from ssa_fwd */
  float* delta;         /* workspace [B, Hq, N] fp32: rowsum(dout * out) */
  float* partials;      /* workspace, ssa_bwd_partials_count() fp32 */
  float* dn;            /* device fp32 scalar, written: dL/dn */
  float* db;            /* device fp32 scalar, written: dL/db */
  const float* ssa_n;
  const float* ssa_b;
  int32_t batch, heads_q, heads_kv, seqlen, head_dim;
  int32_t dtype;
  int32_t causal;
  float softmax_scale;
  void* ds_workspace;   /* optional (NULL: dq recomputes the scores), 16-byte
                           aligned, ssa_bwd_ds_workspace_bytes() bytes; when
                           set, dkdv stores dS' there and dq reads it back, so
                           both steps must get the same pointer.  Packed
                           sequences (ssa_varlen_bwd) need
                           ssa_varlen_bwd_ds_workspace_bytes() bytes.  The
                           vector-ALU kernels (fp32; head dim 256) ignore it:
                           their dq always recomputes. */
} ssa_bwd_args;

/* Library ABI version (SSA_ABI_VERSION). */
int32_t ssa_abi_version(void);

/* Human-readable text of a status code (static storage). */
const char* ssa_status_string(int32_t status);

/* Number of fp32 elements the `partials` workspace of ssa_bwd needs. */
int64_t ssa_bwd_partials_count(int32_t batch, int32_t heads_kv, int32_t seqlen);

/*
 * Bytes of the optional dS' workspace of ssa_bwd: -dS' = P (.) (Delta - dP) /
 * (1 + b|s|) in the input dtype (its contents are private to the dk/dv and dq
 * launches of one backward), per (batch, q-head) the 32-query x 16-key tiles of the
 * causal triangle (all tiles without the mask), 2 * N^2 bytes + O(N) per head
 * causal, 4 * N^2 without.  With it, dk/dv writes dS' and dq becomes one
 * streaming product dS' K instead of a recompute of the scores (the
 * reference recomputes: ssa_triton_kernel.py:408-481, 638-719).  No
 * reference counterpart.
 */
int64_t ssa_bwd_ds_workspace_bytes(int32_t batch, int32_t heads_q, int32_t seqlen, int32_t causal);

/*
 * Forward: out = softmax_rows(t(scale q k^T) [masked]) v, plus the base-2 row
 * normaliser m.  Replaces ssa_flash_attn_forward / _ssa_attn_fwd of
 * training/train/train_ssa_triton/SSA/ssa_triton_kernel.py:732-792 (launch) and
 * :40-260 (kernel).
 */
int32_t ssa_fwd(const ssa_fwd_args* args, void* stream);

/*
 * Backward: delta = rowsum(dout * out), then dk/dv (+ dn/db partials) and dq
 * with recompute from m, then a fixed-order reduction of the partials into
 * dn and db.  Replaces ssa_flash_attn_backward of ssa_triton_kernel.py:795-897
 * (kernels :267-298, :305-481, :488-719 and the two torch .sum() calls at
 * :894-895).
 */
int32_t ssa_bwd(const ssa_bwd_args* args, void* stream);

/*
 * Only the first step of ssa_bwd: delta = rowsum(dout * out) in fp32.
 * Replaces _ssa_attn_bwd_preprocess (ssa_triton_kernel.py:267-298, launched at
 * :827-840).  Reads args->out, args->dout, writes args->delta; other fields
 * unused except the shape/dtype fields.
 */
int32_t ssa_bwd_preprocess(const ssa_bwd_args* args, void* stream);

/*
 * The individual steps of ssa_bwd, for callers that schedule or time them
 * separately.  Each takes the full ssa_bwd_args and must run in this order on
 * one stream: preprocess, dkdv, dq, reduce.
 *  - ssa_bwd_dkdv: dk, dv and the dn/db partials (reads delta).  Replaces
 *    Part 1 of _ssa_attn_bwd + _ssa_attn_bwd_dkdv (ssa_triton_kernel.py:305-401,
 *    545-636).
 *  - ssa_bwd_dq: dq (reads delta).  Replaces Part 2 of _ssa_attn_bwd +
 *    _ssa_attn_bwd_dq (ssa_triton_kernel.py:408-481, 638-719).
 *  - ssa_bwd_reduce: dn, db from the partials in a fixed order.  Replaces
 *    dn_partial.sum() / db_partial.sum() (ssa_triton_kernel.py:894-895).
 */
int32_t ssa_bwd_dkdv(const ssa_bwd_args* args, void* stream);
int32_t ssa_bwd_dq(const ssa_bwd_args* args, void* stream);
int32_t ssa_bwd_reduce(const ssa_bwd_args* args, void* stream);

/*
 * ssa_bwd for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference.  Same arguments and results as ssa_bwd, but
 * args->delta, args->partials and args->ds_workspace are ignored: Delta and
 * the dn/db partials live in a static device array of
 * SSA_NOALLOC_SCRATCH_BYTES bytes that the library holds on every device it
 * runs on until the process ends, and dq recomputes the scores (no dS'
 * workspace).  Needs round256(4 * batch * heads_q * seqlen) +
 * 8 * batch * heads_kv * ceil(seqlen / 128) bytes of it (B=4, H=16, S=4096:
 * about 1 MiB); larger problems return SSA_ERR_SCRATCH with nothing
 * launched.  Calls no allocating routine.  Every call on a device shares that
 * device's array: calls in flight at the same time on one device (on
 * different streams) race; calls in stream order do not.  The first call on
 * each device looks the array's address up (hipGetSymbolAddress): make it
 * outside graph capture; later calls may be captured (they launch kernels
 * only, no memset or copy nodes).
 */
#define SSA_NOALLOC_SCRATCH_BYTES (16ll << 20)
int32_t ssa_bwd_noalloc(const ssa_bwd_args* args, void* stream);

/*
 * Packed (varlen) sequences.  q/k/v/out (and dout/dq/dk/dv) are token streams
 * [total_tokens, heads, head_dim]: an ssa_tensor4 whose stride_b is ignored,
 * stride_h is the head stride and stride_s the token stride.  cu_seqlens is a
 * DEVICE array of batch + 1 int32 offsets (cu[0] = 0, nondecreasing,
 * cu[batch] = total_tokens); document i = tokens [cu[i], cu[i+1]), and
 * attention (causal or not) stays inside each document.  `seqlen` is the
 * length of the longest document (max_seqlen).  m and delta are
 * [heads_q, total_tokens] fp32; partials need
 * ssa_bwd_partials_count(batch, heads_kv, seqlen) floats.  The table is read
 * on the device only: entries are clamped to [0, total_tokens] and lengths to
 * seqlen, so a malformed table gives wrong results but no out-of-bounds
 * access.  `seqlen` must cover the longest document: a longer one is cut to
 * its first `seqlen` tokens.  Token rows that no document covers (before
 * cu[0], from cu[batch] on, the cut tail of a longer document) are written
 * too: out rows 0 and m = -inf by ssa_varlen_fwd, dq / dk / dv rows 0 by
 * ssa_varlen_bwd, so no output keeps stale memory.  No reference
 * counterpart: the reference rejects packed sequences
 * (training/train/train_ssa_triton/SSA/ssa_triton_attention.py:154-156); the
 * layout is Megatron's PackedSeqParams (cu_seqlens_q, max_seqlen_q) as built
 * by training/finetune/nemo_patch/data/packed_sequence.py:116-244.
 */
typedef struct {
  ssa_fwd_args dense;          /* batch = documents, seqlen = max_seqlen */
  const int32_t* cu_seqlens;   /* device, batch + 1 entries */
  int32_t total_tokens;
} ssa_varlen_fwd_args;

typedef struct {
  ssa_bwd_args dense;          /* batch = documents, seqlen = max_seqlen */
  const int32_t* cu_seqlens;   /* device, batch + 1 entries */
  int32_t total_tokens;
} ssa_varlen_bwd_args;

int32_t ssa_varlen_fwd(const ssa_varlen_fwd_args* args, void* stream);
int32_t ssa_varlen_bwd(const ssa_varlen_bwd_args* args, void* stream);

/*
 * Bytes of the optional dS' workspace of ssa_varlen_bwd (dense.ds_workspace):
 * document i (first token s, length L) keeps its heads' tiles from slot
 * s / 32 + i on, a slot holding heads_q * (ceil(max_seqlen / 32) + 1) 1 KB
 * tiles causal (2 * ceil(max_seqlen / 32) without the mask), so the bound
 * (total_tokens / 32 + batch) slots holds any table, however its documents
 * are laid out.  0 for invalid sizes.  No reference counterpart (as
 * ssa_bwd_ds_workspace_bytes).
 */
int64_t ssa_varlen_bwd_ds_workspace_bytes(int32_t batch, int32_t heads_q, int32_t max_seqlen, int32_t total_tokens,
                                          int32_t causal);

/*
 * Decode: one new query token per sequence against a KV cache.  Sequence b
 * attends cache rows 0 .. L_b - 1, L_b = cache_seqlens[b] (a DEVICE int32
 * array, clamped to [0, capacity] on the device); the caller has already
 * written the new token's key and value at row L_b - 1.  The result equals
 * the last row of the causal ssa_fwd over the first L_b rows (out and m; an
 * empty cache gives out = 0, m = -inf).  q and out are [B, Hq, 1, D] views
 * (stride_s unused), the caches [B, Hkv, capacity, D] views with the usual
 * layout rules.  The keys are split into num_splits ranges (0: the library's
 * choice, ssa_decode_num_splits()); with more than one split the partial
 * results go through `workspace` and a second kernel combines them in a fixed
 * order.  No reference counterpart: the reference's generation loop re-runs
 * the full prefix per token (training/train/train_ssa_triton/generate_triton.py:315-331);
 * the math is the forward's (ssa_triton_kernel.py:95-122).
 */
typedef struct ssa_decode_args {
  ssa_tensor4 q;        /* [B, Hq, 1, D] */
  ssa_tensor4 k_cache;  /* [B, Hkv, capacity, D] */
  ssa_tensor4 v_cache;  /* [B, Hkv, capacity, D] */
  ssa_tensor4 out;      /* [B, Hq, 1, D], written */
  float* m;             /* optional (NULL: not written) [B, Hq] contiguous fp32 */
  const int32_t* cache_seqlens;  /* device, batch entries */
  const float* ssa_n;
  const float* ssa_b;
  int32_t batch, heads_q, heads_kv, capacity, head_dim;
  int32_t dtype;
  int32_t num_splits;   /* >= 0; 0 = library choice */
  float softmax_scale;
  void* workspace;      /* ssa_decode_workspace_bytes() bytes, 16-byte aligned;
                           may be NULL when that is 0 (one split) */
} ssa_decode_args;

/* Key splits ssa_decode uses for num_splits = `requested` (0 = library
   choice: about 256 workgroups, splits of at least 256 keys); 0 on invalid
   arguments. */
int32_t ssa_decode_num_splits(int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t capacity,
                              int32_t requested);

/* Workspace bytes of ssa_decode: about (head_dim + 2) fp32 per (batch,
   q-head, split) when it uses more than one split, else 0; 0 on invalid
   arguments. */
int64_t ssa_decode_workspace_bytes(int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t capacity,
                                   int32_t head_dim, int32_t requested);

int32_t ssa_decode(const ssa_decode_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SSA_MI355X_H */
