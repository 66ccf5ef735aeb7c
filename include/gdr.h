/*
 * gdr.h -- C ABI of the MI355X (gfx950) chunkwise gated delta-rule attention library (libgdr.so).
 *
 * One op family, four variants, two modes:
 *   variant  KDA       S_t = diag(e^{g_t}) S_{t-1};  u_t = beta_t (v_t - k_t S_t);  S_t += k_t^T u_t;  o_t = scale q_t S_t
 *            GDN       same with one scalar log-gate per (b, h, t)
 *            GLA       S_t = diag(e^{g_t}) S_{t-1} + k_t^T v_t;  o_t = scale q_t S_t           (no beta, no delta rule)
 *            DELTANET  KDA without decay                                                     (no gate)
 *   mode     chunk     chunkwise-parallel prefill (WY form, chunk = 64 tokens)
 *            recurrent token-by-token recurrence with the state in registers (decode, T = 1 typical)
 *
 * Layouts follow the reference op API: q, k [B, H, T, K]; v, o [B, H, T, V]; gate [B, H, T, K] (KDA, GLA) or
 * [B, H, T] (GDN); beta [B, H, T]; states [N, H, K, V] fp32 row-major with V contiguous.  Every [B, H, T, D]
 * operand is passed as a strided view (element strides for b, h, t; the last dimension must be contiguous),
 * so transposed [B, T, H, D] storage needs no copy.
 *
 * Conventions shared by every entry point:
 *   - All pointers are device pointers, allocated by the caller.  The library allocates nothing and never throws
 *     across this boundary; the only device memory it keeps between calls is the fixed scratch array of
 *     gdr_chunk_fwd_noalloc (on each GPU where that entry point has run).
 *   - Work is enqueued asynchronously on `stream`; no entry point synchronises the device.
 *   - Inputs are never written.  `h0` may alias `ht` (in-place state update); no other aliasing is allowed.
 *   - Return value: GDR_OK (0), or a negative gdr_status.  gdr_last_error() returns a thread-local message
 *     describing the last failure of the calling thread.
 *   - Entry points are re-entrant and thread-safe (gdr_chunk_fwd_noalloc: calls that overlap in time on one GPU share
 *     its scratch and must be serialised by the caller).
 */
#ifndef GDR_H
#define GDR_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GDR_ABI_VERSION 8

typedef enum gdr_variant { GDR_KDA = 0, GDR_GDN = 1, GDR_GLA = 2, GDR_DELTANET = 3 } gdr_variant;

typedef enum gdr_dtype { GDR_F32 = 0, GDR_BF16 = 1, GDR_F16 = 2 } gdr_dtype;

typedef enum gdr_status {
  GDR_OK = 0,
  GDR_ERR_INVALID = -1,     /* bad pointer, shape, stride, dtype or alignment */
  GDR_ERR_UNSUPPORTED = -2, /* valid request this build does not implement (e.g. head dim 96) */
  GDR_ERR_HIP = -3          /* a HIP runtime call failed (launch error) */
} gdr_status;

/* A strided [B, H, T, D] (or [B, H, T] for gate/beta of scalar-gated variants) view.  Strides in elements. */
typedef struct gdr_tensor {
  const void* ptr;
  int32_t dtype; /* gdr_dtype */
  int32_t reserved;
  int64_t stride_b, stride_h, stride_t;
} gdr_tensor;

typedef struct gdr_args {
  int32_t abi_version; /* must equal GDR_ABI_VERSION */
  int32_t variant;     /* gdr_variant */
  int32_t batch;       /* B; must be 1 when cu_seqlens is given */
  int32_t heads;       /* H */
  int32_t seq_len;     /* T (total packed length when cu_seqlens is given) */
  int32_t key_dim;     /* K */
  int32_t value_dim;   /* V */
  float scale;         /* multiplies q; the Python layer resolves `scale or K**-0.5` */
  gdr_tensor q, k, v;  /* q, k, v: bf16, f16 or f32 */
  gdr_tensor gate;     /* f32; ptr NULL for DELTANET */
  gdr_tensor beta;     /* f32; ptr NULL for GLA */
  gdr_tensor out;      /* written; dtype bf16, f16 or f32 */
  const float* h0;     /* [N, H, K, V] f32 contiguous, or NULL for a zero initial state */
  float* ht;           /* [N, H, K, V] f32 contiguous, or NULL when the final state is not wanted */
  const int32_t* cu_seqlens; /* device int32 [n_seqs + 1] packed-sequence offsets, or NULL: cu[0] = 0,
                                non-decreasing, cu[n_seqs] = T (a sequence may be empty: its final state is its
                                initial state) */
  int32_t n_seqs;            /* number of packed sequences (N); ignored when cu_seqlens is NULL (N = B) */
  int32_t reserved;
  void* workspace;           /* chunk mode: device scratch of gdr_chunk_workspace_bytes(args) bytes, 256-aligned;
                                NULL selects the single-launch fused kernel, which needs none (and is slower) */
  int64_t workspace_bytes;   /* size of `workspace` */
} gdr_args;

/* Chunkwise forward (prefill).  Replaces, for all four variants, the forward of
 *   ChunkKimiDeltaAttention     src/ops/kimi_delta_attention.py:535-558
 *   ChunkGatedDeltaNet          src/ops/gated_deltanet.py:395-416
 *   ChunkGatedLinearAttention   src/ops/gated_linear_attention.py:362-384
 *   ChunkDeltaNet               src/ops/deltanet.py:326-347
 * (pad_sequence + chunk_cumsum + kernel matrices + WY representation + state scan + output, six launches and
 * a [B,H,NC+1,K,V] States buffer in the reference).  With a workspace it is two launches on `stream`: a
 * chunk-parallel preparation kernel that writes one record per (chunk, head) into the workspace, then the state
 * scan that reads them; with workspace NULL it is one slower launch that needs no scratch.  On that path q, k, v
 * are all bf16 or all f16 (the MFMA operand type; the Python layer casts), K is 64 or 128 and V a multiple of 64.
 * Two kinds of call take the sequential path instead -- one launch of the recurrent kernel over every token of each
 * sequence, the state, every product and every sum in fp32, no workspace used: q, k, v all f32 (the reference's
 * kernels take f32 dot operands for f32 inputs), and K in {32, 192, 256} (key dims the chunk kernels are not built
 * for; the reference's chunk kernels take any multiple of 64), with q, k, v all bf16 or all f32 and V a multiple of
 * 32.  out may be bf16, f16 or f32.  Any T >= 0, and packed varlen input through cu_seqlens on both paths. */
int gdr_chunk_fwd(const gdr_args* args, hipStream_t stream);

/* Fused layer prologue for gdr_chunk_fwd_fused: the per-token work the reference's KDA layer does in PyTorch before
 * calling the op (src/layers/kimi_delta_attention.py:45-49), done inside the chunk-parallel preparation kernel
 * instead, so the fp32 [B, T, H, K] gate and the normalised q, k never exist in HBM. */
#define GDR_PRO_NORM_QK 1      /* q, k are L2-normalised per (token, head): x / max(||x||_2, 1e-12) (F.normalize) */
#define GDR_PRO_BETA_LOGITS 2  /* beta holds logits; the kernel applies the sigmoid */
#define GDR_PRO_GATE_LOWRANK 4 /* KDA, GLA: gate = -exp(a_log[h]) * softplus(z W[h]^T + bias[h]) in the kernel,
                                  from the rank-R activations z of the gate's first projection; args->gate must
                                  be NULL */
#define GDR_PRO_CONV 8         /* q, k, v are the short convolutions' inputs (q_proj(x), k_proj(x), v_proj(x)): the
                                  kernel applies each depthwise causal convolution (width conv_size) and the SiLU
                                  (ShortConvolution, src/layers/short_convolution.py:11-20) before the
                                  normalisation, with each sequence's conv state */
typedef struct gdr_prologue {
  int32_t flags;            /* GDR_PRO_* bits */
  int32_t rank;             /* R: width of z, a multiple of 32 up to 512 (GATE_LOWRANK) */
  gdr_tensor gate_lowrank;  /* z [B, T, R] bf16 (stride_h ignored; rows 16-byte aligned): decay_proj[0](x) */
  const void* gate_weight;  /* [H * K, R] bf16 row-major, 16-byte aligned: decay_proj[1].weight */
  const float* gate_bias;   /* [H * K] f32, 16-byte aligned, or NULL: decay_proj[1].bias */
  const float* a_log;       /* [H] f32: A_log */
  int32_t conv_size;        /* CONV: the convolutions' width W, 2 to 8 (4, the layer's default, has its own build) */
  int32_t conv_reserved;
  const void* conv_weight[3];    /* CONV: q, k, v weights [H * D, W] bf16 (nn.Conv1d weight [C, 1, W]), 16-byte
                                    aligned; D = K for q, k and V for v */
  const void* conv_state_in[3];  /* CONV: [N, H * D, W - 1] bf16, the W - 1 inputs before each sequence, or NULL
                                    (zeros) */
  void* conv_state_out[3];       /* CONV: [N, H * D, W - 1] bf16, the last W - 1 inputs of each sequence, or NULL;
                                    must not alias conv_state_in.  A sequence of length 0 leaves its entry
                                    untouched. */
} gdr_prologue;

/* gdr_chunk_fwd with the fused prologue `pro`.  Replaces the layer-side q/k normalisation, beta sigmoid and gate
 * computation of KimiDeltaAttention.forward (src/layers/kimi_delta_attention.py:45-49) plus the op call (:51-55).
 * With GDR_PRO_NORM_QK, q and k are the un-normalised rows; with GDR_PRO_BETA_LOGITS, beta holds logits.  Needs a
 * workspace (the two-launch path); other limits as gdr_chunk_fwd.  No backward: train through gdr_chunk_fwd. */
int gdr_chunk_fwd_fused(const gdr_args* args, const gdr_prologue* pro, hipStream_t stream);

/* Bytes of device workspace gdr_chunk_fwd needs for `args` (sizes, variant, key/value dims and varlen fields are
 * read; no pointer is dereferenced), or a negative gdr_status.  The workspace holds one record per (chunk, head)
 * that the chunk-parallel preparation kernel writes and the state-scan kernel reads: the reference keeps the
 * same kind of intermediates (gate cumsum, P, A, W, U, States) in tensors it allocates per call
 * (src/ops/kimi_delta_attention.py:540-553).  For B=4, T=4096, H=16, K=V=128 it is 291.5 MB (71,168 bytes per
 * chunk and head).  A packed call with 2 to 512 sequences adds their longest-first order for the state scan
 * (n_seqs int32, rounded up to 256 bytes).  The size does not depend on dtypes; it is 0 for key dims the chunk
 * kernels do not take (the sequential path needs no workspace, and ignores one it is given, as f32 calls do). */
int64_t gdr_chunk_workspace_bytes(const gdr_args* args);

/* Size of the device scratch behind gdr_chunk_fwd_noalloc (128 MiB per GPU). */
#define GDR_NOALLOC_SCRATCH_BYTES (128LL << 20)

/* gdr_chunk_fwd without a workspace and without any allocation: the two-launch path runs on a scratch array of
 * GDR_NOALLOC_SCRATCH_BYTES that the library holds on each GPU it runs on, from the first call on that GPU until the
 * process ends.  It has no counterpart in the reference: it is for callers that cannot allocate device memory --
 * code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.  Calls no hipMalloc, hipFree or
 * allocating library routine.  args->workspace must be NULL; a call whose gdr_chunk_workspace_bytes exceeds
 * GDR_NOALLOC_SCRATCH_BYTES (e.g. more than 1,885 chunk-head records at K = V = 128: B = 1, T = 4096, H = 16 fits)
 * returns GDR_ERR_UNSUPPORTED.  Nothing in the scratch needs clearing: the preparation launch writes every record
 * the scan launch of the same call reads.  All calls on one GPU share its scratch, so calls that overlap in time on
 * one GPU (different streams, threads or processes' shared contexts) race; serialise them.  Otherwise as
 * gdr_chunk_fwd (same kernels, bit-identical results). */
int gdr_chunk_fwd_noalloc(const gdr_args* args, hipStream_t stream);

/* Gradients of gdr_chunk_fwd for gdr_chunk_bwd.  Every tensor has the shape of its forward counterpart;
 * d_query, d_key and d_value are bf16 or f32 (any of them may differ from the forward dtype), d_gate and
 * d_beta are f32.  d_final (the gradient of the final state) may be NULL for zero; d_initial may be NULL when
 * the initial state's gradient is not wanted. */
typedef struct gdr_grads {
  gdr_tensor d_out;       /* in:  [B, H, T, V] bf16, f16 or f32 */
  const float* d_final;   /* in:  [B, H, K, V] f32 contiguous, or NULL */
  gdr_tensor d_query;     /* out: [B, H, T, K] */
  gdr_tensor d_key;       /* out: [B, H, T, K] */
  gdr_tensor d_value;     /* out: [B, H, T, V] */
  gdr_tensor d_gate;      /* out: like gate; ptr NULL for DELTANET */
  gdr_tensor d_beta;      /* out: [B, H, T]; ptr NULL for GLA */
  float* d_initial;       /* out: [B, H, K, V] f32 contiguous, or NULL */
} gdr_grads;

/* Chunkwise backward.  Replaces ChunkKimiDeltaAttention.backward (src/ops/kimi_delta_attention.py:560-622:
 * a forward recompute, then _chunk_intra_backward, _chunk_state_backward, _chunk_backward_dq/_dk,
 * _chunk_backward_wy_representation, _chunk_backward_kernel_matrix and _chunk_gate_gradient, :200-492) and the
 * backward of its twins ChunkGatedDeltaNet (gated_deltanet.py:419), ChunkGatedLinearAttention
 * (gated_linear_attention.py:387) and ChunkDeltaNet (deltanet.py:350).  `args` describes the forward call (its out, ht and
 * workspace fields are ignored); `grads` names the incoming and outgoing gradients.  `workspace` is device scratch
 * of gdr_chunk_bwd_workspace_bytes(args) bytes, 256-aligned.  Same limits as gdr_chunk_fwd, except that packed
 * varlen input (cu_seqlens) is not supported. */
int gdr_chunk_bwd(const gdr_args* args, const gdr_grads* grads, void* workspace, int64_t workspace_bytes,
                  hipStream_t stream);

/* Bytes of device workspace gdr_chunk_bwd needs (no pointer dereferenced), or a negative gdr_status.  It holds,
 * per chunk and head, the forward record, the state entering the chunk and the gradient of the state leaving it
 * (bf16), u and du (bf16): the buffers the reference allocates per call (:540-553, :575-606). */
int64_t gdr_chunk_bwd_workspace_bytes(const gdr_args* args);

/* The chunk forward of a training step, paired with gdr_chunk_bwd_saved: writes out and ht as gdr_chunk_fwd does and
 * leaves in `workspace` (gdr_chunk_bwd_workspace_bytes(args) bytes, 256-aligned, alive until the backward) the
 * forward records, the per-chunk states and u, so that the backward need not recompute them.  The reference's
 * ChunkKimiDeltaAttention.forward (src/ops/kimi_delta_attention.py:534-558) saves only its inputs and its
 * backward recomputes the states (:566-571); the pair here trades that recompute (a prep launch and a state scan)
 * for the workspace's memory, held from forward to backward.  args->workspace must be NULL.  Limits as
 * gdr_chunk_bwd (bf16 q, k, v; no cu_seqlens); out is bf16 or f32.  Results equal gdr_chunk_fwd's bit for bit. */
int gdr_chunk_fwd_train(const gdr_args* args, void* workspace, int64_t workspace_bytes, hipStream_t stream);

/* gdr_chunk_bwd without the forward recompute: `workspace` as gdr_chunk_fwd_train left it, for the same args
 * (the same tensors, unchanged since).  Gradients equal gdr_chunk_bwd's bit for bit. */
int gdr_chunk_bwd_saved(const gdr_args* args, const gdr_grads* grads, void* workspace, int64_t workspace_bytes,
                        hipStream_t stream);

/* Recurrent forward (decode).  Replaces the `_recurrent_forward` Triton launch of
 *   recurrent_kimi_delta_attention     src/ops/kimi_delta_attention.py:666-692 (kernel :38-68)
 *   recurrent_gated_deltanet           src/ops/gated_deltanet.py:497-520 (kernel :29-59)
 *   recurrent_gated_linear_attention   src/ops/gated_linear_attention.py:461-483 (kernel :30-56)
 *   recurrent_deltanet                 src/ops/deltanet.py:423-445 (kernel :30-57)
 * q, k, v must share one dtype, bf16 or f32 (the Python layer widens mixed or f16 inputs to f32, exactly); out may
 * be bf16, f16 or f32.  Supports K in {32, 64, 128, 192, 256} (the reference's kernel takes any power-of-two head
 * dim, :46), V a multiple of 32, any T >= 0 (cu_seqlens must be NULL; packed input runs through gdr_chunk_fwd). */
int gdr_recurrent_fwd(const gdr_args* args, hipStream_t stream);

/* Multi-token verify for speculative decoding: gdr_recurrent_fwd over a block of T tokens (the pending token plus
 * the drafts) that also records each token's state update row u_t (the row added to the state as k_t^T u_t:
 * beta_t (v_t - k_t S_t) for the delta-rule variants, v_t for GLA) into `updates`, f32 [B, H, T, V] contiguous,
 * 16-byte aligned.  With that record gdr_recurrent_commit rebuilds the state after any accepted prefix from the
 * state the block started from, so nothing is cloned before the verify and nothing is replayed after a rejection.
 * Replaces the verify forward of SpeculativeEngine.generate (src/speculative.py:351-356: RecurrentCache.fork, then
 * the chunk op on the block, padded to 64 tokens by src/ops/utils.py:70-72).  args->ht may be NULL or receive the
 * state after all T tokens.  Same dtype rules and limits as gdr_recurrent_fwd. */
int gdr_recurrent_verify(const gdr_args* args, float* updates, hipStream_t stream);

/* State after the first n_b = clamp(accepted[b], 0, T) tokens of a verified block, for each sequence b:
 *     S = h0 (zero when NULL);  for t < n_b:  S = diag(e^{g_t}) S + k_t^T updates[b, :, t]
 * (scalar decay for GDN, none for DeltaNet).  Reads the variant, sizes, k (bf16 or f32), gate and h0 of `args` and
 * writes args->ht (required; may alias h0); q, v, beta, out and scale are ignored.  `accepted` is a device int32 [B]
 * array, or NULL for all T tokens, so an accept count decided on the device never has to reach the host.  With
 * the inputs of the verify call, accepted = T reproduces the final state gdr_recurrent_verify writes bit for bit.
 * Replaces RecurrentCache.commit / rollback plus the replay forward of the accepted prefix
 * (src/cache.py:59-86, src/speculative.py:397, 425-449). */
int gdr_recurrent_commit(const gdr_args* args, const float* updates, const int32_t* accepted, hipStream_t stream);

/* One speculative cycle in one pass over the state: gdr_recurrent_commit(prev, prev_updates, accepted), which writes
 * the committed state to prev->ht (may alias prev->h0), then gdr_recurrent_verify(args, updates) from that state,
 * which must be args->h0 (== prev->ht).  Bit-identical to the two calls in sequence; the state is read once and
 * held in registers for both, so a cycle streams it once each way instead of twice in and once out.  The previous
 * block (k, gate, record, length) may differ from the new one in T only; its k has the new block's q/k/v dtype.
 * `updates` must not overlap `prev_updates`, and args->ht (optional) must not overlap prev->ht.  Replaces the
 * accept step of the previous cycle together with the verify forward of the next (src/speculative.py:351-356,
 * 397, 425-449; src/cache.py:59-86). */
int gdr_recurrent_commit_verify(const gdr_args* prev, const float* prev_updates, const int32_t* accepted,
                                const gdr_args* args, float* updates, hipStream_t stream);

/* Causal softmax attention of the hybrid stack's attention layer (grouped-query), forward and backward. */
typedef struct gdr_attention_args {
  int32_t abi_version;       /* must equal GDR_ABI_VERSION */
  int32_t batch;             /* B; must be 1 when cu_seqlens is given */
  int32_t heads;             /* query heads H */
  int32_t kv_heads;          /* key/value heads; divides H (query head h reads key/value head h / (H / kv_heads)) */
  int32_t seq_len;           /* T (total packed length when cu_seqlens is given) */
  int32_t head_dim;          /* D: 64 or 128 */
  float scale;               /* softmax scale; the Python layer resolves `softmax_scale or D ** -0.5` */
  int32_t n_seqs;            /* number of packed sequences; ignored when cu_seqlens is NULL */
  gdr_tensor q, k, v;        /* [B, H, T, D] and [B, kv_heads, T, D] views, one dtype (bf16 or f16), rows 16-byte
                                aligned */
  gdr_tensor out;            /* [B, H, T, D], the dtype of q */
  const int32_t* cu_seqlens; /* device int32 [n_seqs + 1] packed-sequence offsets, or NULL */
  float* lse;                /* device fp32 [B][H][T], 4-byte aligned, or NULL.  Forward: when not NULL, receives
                                each query row's log-sum-exp of its scaled scores in log2 units,
                                log2 sum_s 2^(scale log2(e) q.k_s), for the backward.  Backward: the forward's,
                                read. */
} gdr_attention_args;

/* O = softmax(scale Q K^T + causal mask) V per (sequence, query head), with attention confined to each packed
 * sequence when cu_seqlens is given.  Replaces the forward of FlashAttention (src/ops/flash_attention_2.py:161-179,
 * kernel :24-71, reached from src/layers/attention.py:113), which takes no packed input: the reference pads
 * batches (flash_attention_2.py:155-158).  Supports D in {64, 128}, any T >= 1. */
int gdr_attention_fwd(const gdr_attention_args* args, hipStream_t stream);

/* Gradients of gdr_attention_fwd. */
typedef struct gdr_attention_grads {
  int32_t abi_version; /* must equal GDR_ABI_VERSION */
  int32_t reserved;
  gdr_tensor d_out;    /* [B, H, T, D], the dtype of q, rows 16-byte aligned */
  gdr_tensor d_q;      /* [B, H, T, D], the dtype of q, rows 16-byte aligned; written */
  gdr_tensor d_k, d_v; /* [B, kv_heads, T, D], the dtype of q, rows 16-byte aligned; written, each summed over the
                          query heads of its group */
  float* delta;        /* device fp32 [B][H][T] scratch, 4-byte aligned: rowsum(out * d_out), written and then read
                          by the call */
} gdr_attention_grads;

/* dQ, dK, dV of O = softmax(scale Q K^T + causal mask) V given dO.  `args` is the forward call's (q, k, v, out, the
 * lse it wrote, scale, cu_seqlens).  Replaces FlashAttention.backward (src/ops/flash_attention_2.py:180-207: the
 * delta preprocessing :63-75, the dK/dV kernel :77-117 and the dQ kernel :119-151).  Two launches on `stream`: per
 * 128-row query block the row sums delta and dQ, then per 64-row key block of a key/value head dK and dV over every
 * query of its group's heads from the diagonal on.  Supports what gdr_attention_fwd supports. */
int gdr_attention_bwd(const gdr_attention_args* args, const gdr_attention_grads* grads, hipStream_t stream);

/* Depthwise causal convolution + SiLU of the layers' short convolution, segment-aware. */
typedef struct gdr_conv_args {
  int32_t abi_version;       /* must equal GDR_ABI_VERSION */
  int32_t batch;             /* B; must be 1 when cu_seqlens is given */
  int32_t seq_len;           /* T (total packed length when cu_seqlens is given) */
  int32_t channels;          /* C */
  int32_t kernel_size;       /* W, 2 to 8 */
  int32_t n_seqs;            /* number of packed sequences; ignored when cu_seqlens is NULL */
  int32_t apply_silu;        /* nonzero: out = silu(conv(x)) (the layer's form); zero: out = conv(x) */
  int32_t reserved;
  gdr_tensor x;              /* [B, T, C] view (stride_h ignored), channels contiguous */
  gdr_tensor out;            /* [B, T, C] view, channels contiguous */
  const void* weight;        /* [C, W] in x's dtype: nn.Conv1d(C, C, W, groups=C).weight viewed as [C, W] */
  const void* state_in;      /* [N, C, W - 1] in x's dtype: the W - 1 inputs before each sequence, or NULL (zeros) */
  void* state_out;           /* [N, C, W - 1]: the last W - 1 inputs of each sequence after the call, or NULL; must
                                not alias state_in.  The entry of a sequence of length 0 is not written (a caller
                                that wants it unchanged copies state_in there first) */
  const int32_t* cu_seqlens; /* device int32 [n_seqs + 1], or NULL (N = B): cu[0] = 0, non-decreasing,
                                cu[n_seqs] = T; tokens past cu[n_seqs] are not computed */
} gdr_conv_args;

/* out[t, c] = act(sum_{j < W} weight[c, j] x[t - W + 1 + j, c]), where inputs before a sequence's first token come
 * from state_in (or are zero) -- never from the previous packed sequence.  T == 0 is a no-op (pointers unused).  Replaces ShortConvolution.forward
 * (src/layers/short_convolution.py:11-20), whose padded conv runs across the batch layout and has no notion of packed
 * sequences (:9, :15), including its conv-state path (:16-19). */
int gdr_short_conv_fwd(const gdr_conv_args* args, hipStream_t stream);

/* Output epilogue of the KDA layer: out = weight * rmsnorm(x) * silu(gate) over each (token, head) row of V
 * values, where rmsnorm(x) = x / sqrt(mean(x^2) + eps) computed in fp32 and rounded to x's dtype, silu(gate) is
 * rounded to gate's dtype, and the products are taken in out's dtype (f32 when the weight is f32, as PyTorch's type
 * promotion gives; else x's dtype, rounded after each product). */
typedef struct gdr_norm_gate_args {
  int32_t abi_version;       /* must equal GDR_ABI_VERSION */
  int32_t batch;             /* B */
  int32_t seq_len;           /* T */
  int32_t heads;             /* H */
  int32_t value_dim;         /* V: 64, 128, 192 or 256 */
  int32_t weight_dtype;      /* gdr_dtype of weight: GDR_F32 or x's dtype */
  float eps;
  int32_t reserved;
  gdr_tensor x;              /* [B, T, H, V] view of the op's output (stride_b, stride_t, stride_h; unit stride
                                along V; base and strides 16-byte aligned, as for gate and out): bf16, f16 or f32 */
  gdr_tensor gate;           /* [B, T, H, V] view of the output gate's pre-activation, x's dtype */
  gdr_tensor out;            /* [B, T, H, V] view: f32 when weight_dtype is GDR_F32, else x's dtype */
  const void* weight;        /* [V]: the RMSNorm weight */
} gdr_norm_gate_args;

/* Replaces `self.norm(out.transpose(1, 2)) * F.silu(self.output_gate_proj(x).view(...))` of
 * KimiDeltaAttention.forward (src/layers/kimi_delta_attention.py:58-59; RMSNorm src/layers/rmsnorm.py:11-16) with one
 * HBM-bound pass; the gate's two projections stay with the caller (GEMMs). */
int gdr_norm_gate_fwd(const gdr_norm_gate_args* args, hipStream_t stream);

/* Thread-local description of the calling thread's last failure ("" if none).  No reference counterpart:
 * the reference surfaces failures as Python exceptions raised by Triton. */
const char* gdr_last_error(void);

/* GDR_ABI_VERSION of the loaded library, so a binding can refuse a mismatched build. */
int gdr_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* GDR_H */
