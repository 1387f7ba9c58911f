/*
 * decide_hip.h - C ABI of libdecide_hip.so, the MI355X (gfx950) encoder
 * forward for jmwri/decide.
 *
 * The library replaces the reference's GPU stack for inference
 * (internal/cuda: purego driver FFI + NVRTC-built PTX, internal/gpunn:
 * orchestration, cmd/ptxgen: codegen) and gives a device engine for the CPU
 * forward in internal/nn. A host binding (the Go/purego package go/hipnn,
 * the Python ctypes veneer decide_amd/) dlopens it with RTLD_NOW|RTLD_GLOBAL
 * as internal/cuda/lib_unix.go:7-9 does for libcuda.
 *
 * Conventions (mirroring internal/cuda/driver.go):
 *   - every call returns an int status; 0 is success (driver.go:123-142);
 *   - a missing or unusable GPU yields DN_NO_GPU, which the binding maps to
 *     the reference's ErrNoGPU sentinel and its CPU fallback
 *     (driver.go:19, :157-167; internal/train/engine.go:42-61);
 *   - on failure dn_last_error() names the operation and cause;
 *   - host arrays are caller-owned and copied synchronously; device memory
 *     is owned by the context and freed by dn_close;
 *   - one context is single-stream and not re-entrant: callers serialise
 *     calls, as decide.Local does with its fmu mutex (local.go:193-194).
 *
 * All pointers named d_* are device pointers; all others are host pointers.
 */
#ifndef DECIDE_HIP_H
#define DECIDE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DN_ABI_VERSION 1

enum {
  DN_OK = 0,
  DN_NO_GPU = 1,        /* no HIP device / runtime: fall back to the CPU */
  DN_INVALID_ARG = 2,   /* malformed input; message mirrors forward.go */
  DN_OUT_OF_MEMORY = 3,
  DN_DEVICE_ERROR = 4,  /* a HIP call or kernel failed */
  DN_UNSUPPORTED = 5    /* geometry or mode this build does not implement */
};

enum { DN_PRECISION_FP32 = 0, DN_PRECISION_BF16 = 1, DN_PRECISION_FP16 = 2 };

typedef struct dn_ctx dn_ctx;

/* ABI version of the loaded library (DN_ABI_VERSION). */
int dn_abi_version(void);

/* Human-readable name of a status code. */
const char *dn_status_string(int status);

/* Opens device `device` and creates a context.
 * Replaces cuda.Open (internal/cuda/driver.go:157-191): DN_NO_GPU when the
 * HIP runtime reports no device (driver.go:157-167). */
int dn_open(int device, dn_ctx **out);

/* Frees every device allocation of the context.
 * Replaces gpunn.(*Model).Free + cuda.(*Device).Close (engine.go:166). */
void dn_close(dn_ctx *ctx);

/* Message of the last failed call on ctx ("" if none); valid until the next
 * call on ctx. Counterpart of cuda.Error.Error (driver.go:123-136). */
const char *dn_last_error(const dn_ctx *ctx);

/* Runs the context's work on `stream` (a hipStream_t; NULL is the default
 * stream) instead of the context's own non-blocking stream.
 * No counterpart in the reference (CUDA's context stream was implicit). */
int dn_set_stream(dn_ctx *ctx, void *stream);

/* Model geometry, the fields of nn.Config (internal/nn/config.go:12-27;
 * defaults from LoadConfig :33-95) plus the arithmetic mode:
 * DN_PRECISION_BF16 = bf16 GEMM/attention operands, fp32 accumulate,
 * residual stream, statistics and head; DN_PRECISION_FP16 = the same with
 * IEEE binary16 operands (11-bit significand where bf16 has 8: projection
 * weights rounded to nearest fp16, activations stored in fp16; same MFMA
 * rate and bytes; inference only; a projection weight of magnitude >= 65520
 * gives DN_UNSUPPORTED); DN_PRECISION_FP32 = fp32 MFMA everywhere (the
 * validation build). Must precede dn_upload_tensor.
 * Replaces the config capture of gpunn.New (internal/gpunn/model.go:80-122).
 * head_dim 64 with hidden % 256 == 0 (<= 1024) and inter % 64 == 0
 * (ModernBERT-base: 768/1152/12 heads) runs the MFMA kernels; other
 * geometries with hidden <= 1024, hidden % 8 == 0 and head_dim 8, 16, 32 or
 * 64 (the reference's own test models, e.g. tiny_ref's 32/48/4 heads) run
 * any-shape GEMM and attention kernels (inference only: dn_enable_training
 * reports DN_UNSUPPORTED for them); anything else gives DN_UNSUPPORTED. */
int dn_set_config(dn_ctx *ctx, int hidden, int inter, int heads, int layers, int vocab, float eps,
                  int half_window, double theta_global, double theta_local,
                  const uint8_t *layer_is_sliding /* [layers] */, int precision);

/* Uploads one parameter by its nn.Model.Tensors() name
 * (internal/nn/model.go:51-84), as n float32 values in that tensor's layout.
 * bf16 (fp16) mode converts the four projection matrices to bf16 (fp16),
 * rounding to nearest even, and interleaves the Wi rows for the fused GeGLU
 * epilogue.
 * Replaces the per-tensor upload loop of gpunn.New (model.go:80-122). */
int dn_upload_tensor(dn_ctx *ctx, const char *name, const float *data, int64_t n);

/* The same upload from bfloat16 bits, as a BF16 entry of a safetensors
 * bundle holds them (n uint16 values, little-endian bit patterns). bf16 mode
 * stores the projection matrices' bits as given (no float32 round trip);
 * fp16 mode converts them to binary16 (exact for magnitudes 2^-17 .. 65504);
 * every other tensor, and every tensor in fp32 mode, is widened exactly to
 * float32. Replaces the BF16 branch of safetensors.(*File).Float32
 * (internal/safetensors/safetensors.go:113-124) followed by the upload. */
int dn_upload_tensor_bf16(dn_ctx *ctx, const char *name, const uint16_t *bits, int64_t n);

/* 1 when every tensor the configured model needs has been uploaded. */
int dn_weights_ready(const dn_ctx *ctx);

/* Encoder + scorer forward over a batch of packed sequences, returning one
 * logit per mask position in batch order.
 * Replaces nn.(*Model).Forward (internal/nn/forward.go:129-245, inference,
 * trainFrom >= Layers) and gpunn.(*Model).Forward (internal/gpunn/model.go:204-330)
 * including HeadForward (forward.go:250-282), which ran on the host there.
 * The nn.Sequence slice is passed flattened:
 *   seq_len[nseq]            len(Sequence.IDs)
 *   ids[T], pos[T]           Sequence.IDs, Sequence.Pos (T = sum seq_len)
 *   opt_id[T] or NULL        Sequence.OptID; -1 = prefix; a sequence with
 *                            OptID == nil is passed as all -1; NULL = all nil
 *   nmask[nseq], mask_pos[]  Sequence.MaskPos of each sequence, concatenated
 *   logits[logits_cap]       output, sum(nmask) values
 * Validation and messages follow forward.go:145-150, :181-183, :192-196
 * (DN_INVALID_ARG). */
int dn_forward(dn_ctx *ctx, int nseq, const int32_t *seq_len, const int32_t *ids, const int32_t *pos,
               const int32_t *opt_id, const int32_t *nmask, const int32_t *mask_pos, float *logits,
               int logits_cap);

/* The same forward with the token arrays already resident on the device.
 * seq_len is a host array (the batch layout); d_row_tok holds, per output
 * row, the global token index of its mask position. Inputs are trusted to
 * satisfy dn_forward's checks; out-of-range ids or rows are clamped by the
 * kernels and reported by the next dn_check_device_errors. Asynchronous on
 * the context's stream. No separate counterpart in the reference (it is the
 * device part of gpunn.(*Model).Forward, model.go:261-328). */
int dn_forward_device(dn_ctx *ctx, int nseq, const int32_t *seq_len, const int32_t *d_ids,
                      const int32_t *d_pos, const int32_t *d_opt_id, int nrows, const int32_t *d_row_tok,
                      float *d_logits);

/* dn_forward_device without allocating: every buffer the forward works in
 * beyond the weights and the caller's inputs and outputs (activations, batch
 * layout, head scratch) comes from one static 64 MiB device array per GPU, so
 * the call makes no hipMalloc / hipFree. About 5,100 tokens per call fit at
 * ModernBERT-base in bf16 (about 2,900 in fp32); a larger batch gets
 * DN_INVALID_ARG naming the bytes it needs. All calls on one GPU share the
 * array: calls that overlap on one GPU (two contexts or streams) race. The
 * context's stream is synchronised before the batch layout is uploaded, so
 * the call cannot be captured into a graph: on a capturing stream it returns
 * DN_UNSUPPORTED before enqueuing anything. Arguments and results as
 * dn_forward_device. No counterpart in the reference: it is for callers that
 * cannot allocate device memory (tight serving loops, harnesses that forbid
 * hipMalloc). */
int dn_forward_device_noalloc(dn_ctx *ctx, int nseq, const int32_t *seq_len, const int32_t *d_ids,
                              const int32_t *d_pos, const int32_t *d_opt_id, int nrows,
                              const int32_t *d_row_tok, float *d_logits);

/* Synchronises the stream and reports (DN_INVALID_ARG) any out-of-range token
 * id or row index seen by dn_forward_device since the last check. */
int dn_check_device_errors(dn_ctx *ctx);

/* C (M x N) = op(A) (M x K) . op(B) (K x N), adding into C when accumulate
 * is set, with blas.Sgemm semantics (internal/blas/gemm.go:55-63): row-major
 * host arrays with leading dimensions; transA means A is stored K x M,
 * transB means B is stored N x K. Computed on the GPU with fp32 MFMA.
 * Replaces cuda.(*Kernels).Gemm (internal/cuda/kernels.go:52-71). */
int dn_gemm_f32(dn_ctx *ctx, int transA, int transB, int M, int N, int K, const float *A, int lda,
                const float *B, int ldb, float *C, int ldc, int accumulate);

/* Device-resident projection GEMM as the forward runs it:
 * d_C[M x N] (fp32) (+)= d_A[M x K] . d_B[N x K]^T, with operands of the
 * given precision (bf16 or fp32). Requires N % 128 == 0 and K a multiple of
 * 64 (bf16) / 32 (fp32). Asynchronous. Same reference counterpart as
 * dn_gemm_f32 (the NT case, linearFwd forward.go:122-124). */
int dn_gemm_device(dn_ctx *ctx, int precision, int M, int N, int K, const void *d_A, const void *d_B,
                   float *d_C, int accumulate);

/* The same GEMM with the output rounded to the operand type, as the forward
 * stores its QKV projection: d_C[M x N] (bf16 or fp16, row stride N) =
 * d_A[M x K] . d_B[N x K]^T, fp32 accumulate, round to nearest even. 16-bit
 * precisions only; N % 128 == 0, K % 64 == 0. Asynchronous. Same reference
 * counterpart as dn_gemm_device (linearFwd, forward.go:122-124). */
int dn_gemm_device_store(dn_ctx *ctx, int precision, int M, int N, int K, const void *d_A, const void *d_B,
                         void *d_C);

/* Inference forwards (dn_forward, dn_forward_device, dn_evaluate) of batches
 * with at least min_tokens tokens and two or more sequences run in two parts
 * of whole sequences (cut nearest half the tokens; both parts must exceed
 * 1024 tokens), one on the context's stream and one on a second stream
 * of the context (default priority), layer by layer in alternation, joined
 * before the scorer head: one part's kernels fill the GPU around the other's.
 * The logits are the same as the single-stream forward's. 0 turns it off; the
 * default is 8192. While a kernel probe is enabled (dn_set_probe) forwards
 * run on one stream. No counterpart in the reference. */
int dn_set_stream_split(dn_ctx *ctx, int min_tokens);

/* Inference forwards (dn_forward, dn_forward_device, dn_evaluate) of batches
 * with at least min_tokens tokens, at most a quarter of them option rows, run
 * the last encoder layer past its attention on the option rows only: their
 * attention output and residual rows are gathered, and Wo, mlp_norm, Wi and
 * MlpWo run on R rows instead of T. Every step after attention is row-wise and
 * the scorer head reads only those rows, so the logits are those of the full
 * layer up to the summation order of the smaller GEMMs' kernels. 0 turns it
 * off; the default is 2048. While the kernel probe times the last layer
 * (dn_set_probe) forwards run the full layer. No counterpart in the reference
 * (forward.go:212-243 runs every layer over all tokens, then gathers). */
int dn_set_row_tail(dn_ctx *ctx, int min_tokens);

/* bf16 and fp16 inference forwards of more than 1024 tokens (or parts of a two-stream
 * forward) run attn_norm and mlp_norm folded into the GEMMs around them: the
 * residual GEMM before a LayerNorm (Wo, MlpWo) also writes the norm's operand
 * ((x - m) * w in the operand type) of the new residual row x, with m the row mean of the
 * previous LayerNorm and w the norm weight, and per 192 columns the row's
 * (mean, M2) as an fp32 pair (reduced in fp64); the GEMM after it (QKV, Wi)
 * merges those (in fp64) into the row's
 * mean and rstd and computes rstd * (A.B^T - (mean - m) * sum_k w[k] B[n][k]),
 * i.e. LayerNorm(x).B^T, so the LayerNorm launches (a read of the fp32
 * residual stream each) disappear. The logits move by the bf16 rounding of
 * the operand (x - m) * w instead of the normalised row, the same size of
 * error. on = 0 runs the LayerNorm kernels; the default is on. No
 * counterpart in the reference (forward.go:289-294, :324 normalise, then
 * project). */
int dn_set_ln_fold(dn_ctx *ctx, int on);

/* How the small-M GEMM kernel (batches of at most 128 tokens, 16-bit modes,
 * 32 x 32 output tiles) loads its operands: 1 (the default) whole 128-byte
 * rows into LDS by global->LDS DMA, then the MFMA fragments from LDS; 0 each
 * lane's fragment straight into registers. Both feed the same MFMAs the same
 * operands in the same order: the logits are identical. No counterpart in
 * the reference. */
int dn_set_small_m_loads(dn_ctx *ctx, int mode);

/* Certified argmax for the 16-bit modes. The reference answers a question
 * with the argmax of its options' float32 logits (local.go:254-262, :291);
 * a bf16 / fp16 forward moves each logit by its rounding error, so options
 * closer than that error may swap. With margin > 0, every dn_forward and
 * dn_forward_device checks each sequence's logits (dn_evaluate lays out one
 * question per sequence): a sequence whose two largest logits are less than
 * `margin` apart, or with a non-finite logit, is run again on an fp32 twin of
 * the context (same geometry and weights in float32, fp32 MFMA: the
 * validation mode) and its logits are replaced. The margin should bound the
 * 16-bit path's error of a logit difference; measured on ModernBERT-base
 * random-init requests: fp16 1.2e-4 RMS (5e-4 max over 1,000 requests), bf16
 * 1.0e-3 RMS. dn_forward_device becomes synchronous and expects each
 * sequence's rows to be its mask positions (rows are assigned to sequences by
 * token index). Must follow dn_set_config and precede the weight uploads
 * (which then also go to the twin); 0 turns it off. Training contexts and
 * the fp32 mode refuse it; dn_forward_device_noalloc returns the 16-bit
 * logits unchecked. No counterpart in the reference (its GPU path is fp32). */
int dn_set_certify(dn_ctx *ctx, float margin);
/* Sequences checked and recomputed by certification since the last call
 * (then reset to 0). */
int dn_read_certify(dn_ctx *ctx, int64_t *checked, int64_t *recomputed);

/* Waits for the context's stream. */
int dn_synchronize(dn_ctx *ctx);

/* Kernel probe for measurement: while enabled (layer >= 0), every forward
 * records HIP events on the context's stream around the five per-layer
 * launches of encoder layer `layer` (DN_PROBE_* order). dn_read_probe
 * synchronises, adds each launch's duration to ms[5] and the number of
 * forwards seen to *count, and resets the probe. layer < 0 disables it;
 * layer >= 0 creates the events of the next 128 forwards and backwards at once.
 * No counterpart in the reference (its tests time whole calls,
 * internal/cuda/gemm_test.go:141-181). */
enum { DN_PROBE_QKV = 0, DN_PROBE_ATTENTION = 1, DN_PROBE_WO = 2, DN_PROBE_WI = 3, DN_PROBE_MLPWO = 4 };
int dn_set_probe(dn_ctx *ctx, int layer);
int dn_read_probe(dn_ctx *ctx, double *ms /* [5] */, int *count);

/* The same probe in dn_backward: events around three launches of layer
 * `layer`'s backward: the QKV weight-gradient GEMM (split-K GEMM + its
 * reduce, on the weight-gradient stream), the input-gradient GEMM
 * dqkv . Wqkv, and the attention backward (both kernels). dn_read_probe_backward
 * adds their durations to ms[3] and the number of backward passes seen to
 * *count, and resets it. No counterpart in the reference. */
enum { DN_PROBE_BWD_WGRAD_QKV = 0, DN_PROBE_BWD_DGRAD_QKV = 1, DN_PROBE_BWD_ATTENTION = 2 };
int dn_read_probe_backward(dn_ctx *ctx, double *ms /* [3] */, int *count);

/* Attainable MFMA rate of this GPU (TFLOP/s), for the roofline: a
 * register-only loop of v_mfma_f32_32x32x16_bf16 (modes 0, 1),
 * v_mfma_f32_32x32x2_f32 (modes 2, 3: the fp32 validation mode and
 * dn_gemm_f32) or v_mfma_f32_32x32x16_f16 (modes 4, 5) in the projection
 * GEMMs' wave pattern on every CU, no memory traffic. Modes 0, 2 and 4:
 * operands with the forward's statistics (activations ~ N(0,1), weights ~
 * N(0,0.02)) that change every iteration, as a real GEMM's do; modes 1, 3
 * and 5: constant operands. The matrix core runs slower the more its inputs
 * toggle, so modes 0, 2 and 4 are the ceilings a GEMM on real data can
 * approach. Synchronous (~10 ms). No counterpart in the
 * reference. */
int dn_mfma_calibrate(dn_ctx *ctx, int mode, double *tflops);

/* ---- host-side helpers mirroring the reference's scoring glue ---------- */

/* nn.BuildSequence (internal/nn/forward.go:28-56). Writes pos[n] and, when
 * independent and at least one mask token exists, opt_id[n] (*has_opt = 1);
 * mask_pos receives the mask token indices (capacity n). Returns their
 * count. */
int dn_build_sequence(const int32_t *ids, int n, int32_t mask_id, int independent, int32_t *pos,
                      int32_t *opt_id, int32_t *mask_pos, int *has_opt);

/* decide.Local answer post-processing for K logits (local.go:206-262):
 * probs = softmax(logit / max(temperature, 1e-4)) in float64; *choice =
 * argmax of the raw logits (first index wins ties); *confidence =
 * marginConfidence(probs) rounded to 3 places. probs are NOT rounded. */
int dn_answer(const double *logits, int k, double temperature, double *probs, int *choice,
              double *confidence);

/* local.go round(): math.RoundToEven(x * 10^places) / 10^places. */
double dn_round(double x, int places);

/* Question kinds of decide.Local (local.go:264-356). */
enum { DN_KIND_CHOICE = 0, DN_KIND_SCORE = 1, DN_KIND_NOUL = 2 };

/* Answers every question of one SystemOne call with ONE forward over all of
 * them. decide.Local.Evaluate (local.go:126-150) runs evalChoice / evalScore /
 * evalNoul (local.go:264-356) one question at a time, one Forward each; the
 * answers here are those, computed from a single batched Forward.
 * Per question q (inputs):
 *   kind[q]         DN_KIND_*
 *   n_opt[q]        number of options (Choice criteria, Score levels; 2 for
 *                   a Noul)
 *   q_len[q], ids   the tokenizer's ids of bundle.PackText(state,
 *                   instructions, options) with [CLS]/[SEP] (local.go:185-186),
 *                   concatenated over questions; questions that skip the
 *                   model (Choice/Score with n_opt <= 1) may pass q_len 0
 *   temperature[q]  Calibration.TemperatureFor(kind) (bundle.go:39-50)
 *   mask_id, independent: as nn.BuildSequence (Tokenizer.MaskID,
 *                   Meta.IndependentOptions)
 * Outputs: probs[sum n_opt] calibrated probabilities rounded to 4 places
 * (question q's at offset sum of n_opt[<q]); choice[q] argmax of the raw
 * logits for a Choice, else -1; confidence[q] marginConfidence for a Choice
 * or Score, else 0; value[q] the Score's expectation rounded to 2 places or
 * the Noul's p(first option) clamped and rounded to 4 places, else 0. A
 * question with n_opt == 0 gets no probabilities, choice -1, confidence 0.
 * Errors (DN_INVALID_ARG) name the first failing question in order, with
 * rawLogits' messages ("input is N tokens; the limit is 8192", "input
 * contains the reserved [MASK] token"); then nothing is computed. */
int dn_evaluate(dn_ctx *ctx, int nq, const int32_t *kind, const int32_t *n_opt, const int32_t *q_len,
                const int32_t *ids, const double *temperature, int32_t mask_id, int independent, double *probs,
                int32_t *choice, double *confidence, double *value);

/* ---- host tokenizer (internal/tokenizer/tokenizer.go) ------------------ */

/* ModernBERT's byte-level BPE tokenizer: NFC, the GPT-2 pre-tokenizer,
 * added tokens, [CLS] $A [SEP]. Host code only; a tokenizer is safe for
 * concurrent use (as tokenizer.Tokenizer is). Errors are reported through
 * dn_last_error(NULL). */
typedef struct dn_tokenizer dn_tokenizer;

/* Parses tokenizer.json contents (len bytes). Replaces tokenizer.Parse
 * (internal/tokenizer/tokenizer.go:60-130): BPE models only; merges as
 * ["a","b"] pairs or "a b" strings, the first occurrence of a pair keeping
 * its rank; special, non-normalized added tokens match the raw text, the
 * others the normalized text; [CLS], [SEP] and [MASK] must exist. */
int dn_tokenizer_parse(const char *json, int64_t len, dn_tokenizer **out);

void dn_tokenizer_free(dn_tokenizer *tok);

/* Ids of [CLS], [SEP], [MASK] and [PAD] (Tokenizer.ClsID / SepID / MaskID,
 * tokenizer.go:40-50); any pointer may be NULL. */
int dn_tokenizer_special_ids(const dn_tokenizer *tok, int32_t *cls, int32_t *sep, int32_t *mask, int32_t *pad);

/* Tokenizer.Encode (tokenizer.go:133-160) of len bytes of UTF-8 text, with
 * [CLS] ... [SEP] when add_special. *n receives the id count; the ids are
 * written when it is <= cap, else DN_INVALID_ARG (call again with *n). */
int dn_tokenize(dn_tokenizer *tok, const char *text, int64_t len, int add_special, int32_t *ids, int64_t cap,
                int64_t *n);

/* preTokenize (tokenizer.go:214-272): the pieces of text under the GPT-2
 * split rule, as end offsets into the text (invalid UTF-8 bytes count as
 * U+FFFD, three bytes, as Go's []rune conversion makes them). */
int dn_pretokenize(const char *text, int64_t len, int64_t *ends, int64_t cap, int64_t *n);

/* Unicode NFC of UTF-8 text (norm.NFC.String in Encode, tokenizer.go:147),
 * invalid bytes passed through; same output-capacity convention. */
int dn_nfc(const char *text, int64_t len, char *out, int64_t cap, int64_t *n);

/* ---- Training (the device half of internal/gpunn + internal/train's engine).
 * Weights, gradients and AdamW moments of every tensor (encoder and scorer
 * head) live on the device; the loss and learning-rate schedule stay with
 * the caller, as in internal/train/trainer.go:300-330. Gradient and moment
 * tensors use the same names and layouts as dn_upload_tensor. */

/* Enables training on a configured context: from here on, uploads in bf16
 * mode also keep fp32 master weights (AdamW updates them and re-rounds the
 * bf16 operand copy). Must precede the weight uploads. Gradients and
 * moments start at zero. Replaces gpunn.New's per-parameter w/g/m/v
 * buffers (internal/gpunn/model.go:80-121). */
int dn_enable_training(dn_ctx *ctx);

/* Freezes encoder layers below train_from and, unless train_emb, the token
 * embeddings (always frozen when train_from > 0); the embedding norm is
 * frozen when train_from > 0. Replaces gpunn.(*Model).SetTrainable
 * (internal/gpunn/model.go:155-171); the same rules as NewAdamW
 * (internal/train/optim.go:31-65). */
int dn_set_trainable(dn_ctx *ctx, int train_from, int train_emb);

/* Forward that keeps the activations dn_backward needs (for layers >=
 * train_from). Arguments and validation as dn_forward. Replaces
 * gpunn.(*Model).Forward (internal/gpunn/model.go:204-330) and
 * nn.(*Model).Forward with trainFrom < Layers (internal/nn/forward.go:129). */
int dn_forward_train(dn_ctx *ctx, int nseq, const int32_t *seq_len, const int32_t *ids, const int32_t *pos,
                     const int32_t *opt_id, const int32_t *nmask, const int32_t *mask_pos, float *logits,
                     int logits_cap);

/* Accumulates into the device gradients the gradient of a loss whose
 * derivative with respect to the last dn_forward_train's logits is dlogits
 * [nrows]. Head and final norm included; layers below train_from get none;
 * the token embeddings only with train_emb and train_from == 0. Replaces
 * gpunn.(*Model).Backward (internal/gpunn/model.go:384-477) and
 * nn.(*Model).Backward (internal/nn/backward.go:19-115). DN_INVALID_ARG
 * without a preceding dn_forward_train (any other forward invalidates it). */
int dn_backward(dn_ctx *ctx, const float *dlogits, int nrows);

/* Clears every gradient. Replaces gpunn.(*Model).ZeroGrad (model.go:479-486). */
int dn_zero_grad(dn_ctx *ctx);

/* Sum of squares (float64) of the gradients of all trainable tensors;
 * sqrt of it is AdamW.GradNorm (optim.go:68-90) over the whole model.
 * Replaces gpunn.(*Model).GradSumSq (model.go:488-505). */
int dn_grad_sumsq(dn_ctx *ctx, double *out);

/* One AdamW step (beta1 0.9, beta2 0.999, eps 1e-8) on every trainable
 * tensor, gradients first scaled by grad_scale: encoder tensors at lr,
 * scorer tensors at head_lr; decoupled weight decay weight_decay*rate on
 * 2-D tensors except the token embeddings. Replaces
 * gpunn.(*Model).Update (model.go:507-529) + AdamW.Update (optim.go:94-145). */
int dn_adamw_step(dn_ctx *ctx, float lr, float head_lr, float weight_decay, float grad_scale);

enum { DN_STATE_WEIGHT = 0, DN_STATE_GRAD = 1, DN_STATE_M = 2, DN_STATE_V = 3 };

/* Copies one tensor's weights (fp32 masters when training in bf16),
 * gradient or moment into out [n]. Replaces SyncToHost / DownloadGrads /
 * DownloadAdam (internal/gpunn/model.go:531-600). */
int dn_download_tensor(dn_ctx *ctx, const char *name, int which, float *out, int64_t n);

/* Sets one tensor's gradient or moment (DN_STATE_GRAD/M/V) from data [n];
 * with dn_set_adam_step, restores a checkpoint's optimizer state. Replaces
 * UploadAdam (internal/gpunn/model.go:578-593). */
int dn_upload_state(dn_ctx *ctx, const char *name, int which, const float *data, int64_t n);
int dn_set_adam_step(dn_ctx *ctx, int step);

#ifdef __cplusplus
}
#endif

#endif /* DECIDE_HIP_H */
