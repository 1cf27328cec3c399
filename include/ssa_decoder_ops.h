/*
 * Fused element-wise operators of the SSA decoder layer (gfx950), next to the
 * attention path: the callers either side of it in a transformer layer.
 *
 * Same rules as ssa_mi355x.h: the caller owns every buffer, the call only
 * enqueues on `stream` (a hipStream_t, NULL = default stream) and returns a
 * status before any launch when an argument is invalid.
 */
#ifndef SSA_DECODER_OPS_H
#define SSA_DECODER_OPS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  SSA_OPS_OK = 0,
  SSA_OPS_ERR_NULL_POINTER = 1,
  SSA_OPS_ERR_SHAPE = 2,
  SSA_OPS_ERR_DTYPE = 3,
  SSA_OPS_ERR_ALIGNMENT = 4,
  SSA_OPS_ERR_LAUNCH = 5
};

/*
 * Rotary position embedding, rotate-half form, applied to q or k before the
 * core attention.  Replaces the rotary step of the Megatron SelfAttention that
 * the reference's SSA layer spec builds
 * (training/train/train_ssa_triton/SSA/ssa_triton_layer_specs.py:96-127;
 * Megatron's default non-interleaved RoPE, rotary base 10000).
 *
 * x: [seqlen, batch, heads, head_dim] in bf16/fp16 with element strides
 * x_stride_{s,b,h} (stride 1 over head_dim); y: contiguous, same shape.
 * cos, sin: fp32 [seqlen, head_dim / 2], row s = cos / sin of s * inv_freq.
 * inverse = 1 rotates by the negative angle (the backward).  head_dim 64 or
 * 128; x, y 8-byte aligned, strides multiples of 4 elements, tables 16-byte
 * aligned.
 */
typedef struct {
  const void* x;
  int64_t x_stride_s, x_stride_b, x_stride_h;
  void* y;
  const float* cos;
  const float* sin;
  int32_t seqlen, batch, heads, head_dim;
  int32_t dtype; /* 0 = bf16, 1 = fp16 */
  int32_t inverse;
} ssa_rope_args;

int32_t ssa_rope(const ssa_rope_args* args, void* stream);

/*
 * RMSNorm of the decoder layer's input and pre-MLP norms (and the final
 * norm): y = x * (mean(x^2) + eps)^-1/2 * weight over rows of `hidden`
 * values.  Replaces the TE/Megatron RMSNorm modules of the reference's SSA
 * layer spec (training/train/train_ssa_triton/SSA/ssa_triton_layer_specs.py:
 * 96-127; normalization "RMSNorm" in the run configuration).
 *
 * x, weight: fp32 (the residual stream and the parameter), x [rows, hidden]
 * contiguous, 16-byte aligned; hidden a multiple of 4, at most 4096.  y is
 * written in out_dtype (0 bf16, 1 fp16, 2 fp32: the dtype of the next GEMM's
 * input), rstd [rows] fp32 is kept for the backward.  The backward reads dy
 * in dy_dtype, writes dx fp32 [rows, hidden] and dweight fp32 [hidden]; its
 * workspace holds ssa_rmsnorm_workspace_floats(rows, hidden) fp32 partial
 * weight gradients, summed in a fixed order (deterministic).
 */
typedef struct {
  const void* x;
  const void* weight;
  void* y;
  float* rstd;
  int32_t rows, hidden;
  int32_t out_dtype;
  float eps;
} ssa_rmsnorm_fwd_args;

typedef struct {
  const void* x;
  const void* weight;
  const void* dy;
  const float* rstd;
  float* dx;
  float* dweight;
  float* workspace;
  int32_t rows, hidden;
  int32_t dy_dtype;
} ssa_rmsnorm_bwd_args;

int64_t ssa_rmsnorm_workspace_floats(int32_t rows, int32_t hidden);
int32_t ssa_rmsnorm_fwd(const ssa_rmsnorm_fwd_args* args, void* stream);
int32_t ssa_rmsnorm_bwd(const ssa_rmsnorm_bwd_args* args, void* stream);

/*
 * SwiGLU gate of the MLP: h = silu(gate) * up, where z = [gate | up] is the
 * fc1 output, rows of 2 * ffn values.  Replaces the gated-linear-unit
 * activation of the Megatron MLP in the reference's SSA layer spec
 * (training/train/train_ssa_triton/SSA/ssa_triton_layer_specs.py:96-127;
 * "swiglu" in the run configuration).
 *
 * backward = 0: out = h [rows, ffn].  backward = 1: dh [rows, ffn] in, out =
 * dz [rows, 2 * ffn] = [d gate | d up].  bf16 or fp16, contiguous, 8-byte
 * aligned; ffn a multiple of 4.  fp32 math, one rounding per output.
 */
typedef struct {
  const void* z;
  const void* dh;
  void* out;
  int32_t rows, ffn;
  int32_t dtype; /* 0 = bf16, 1 = fp16 */
  int32_t backward;
} ssa_swiglu_args;

int32_t ssa_swiglu(const ssa_swiglu_args* args, void* stream);

/*
 * Cross-entropy of the output layer's logits against integer labels, the
 * loss of the reference's training step (Megatron's GPT loss over the vocab
 * logits; the reference runs it through its layer spec,
 * training/train/train_ssa_triton/SSA/ssa_triton_layer_specs.py:96-127).
 *
 * logits [rows, vocab] bf16/fp16 contiguous, 8-byte aligned, vocab a
 * multiple of 4; labels int64 [rows], a row with a label outside [0, vocab)
 * is ignored (loss 0, gradient 0).  Forward (backward = 0): loss [rows] fp32
 * per row (log-sum-exp minus the label's logit) and lse [rows] fp32, kept for
 * the backward.  Backward (backward = 1): dlogits [rows, vocab] in the logits'
 * dtype = (softmax - one-hot) * scale[0], scale a device fp32 scalar (the
 * upstream gradient over the number of counted rows for a mean).
 */
typedef struct {
  const void* logits;
  const void* labels;
  float* loss;
  float* lse;
  const float* scale;
  void* dlogits;
  int32_t rows, vocab;
  int32_t dtype; /* 0 = bf16, 1 = fp16 */
  int32_t backward;
} ssa_cross_entropy_args;

int32_t ssa_cross_entropy(const ssa_cross_entropy_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SSA_DECODER_OPS_H */
