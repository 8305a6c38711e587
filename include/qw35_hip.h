/* qw35_hip.h — C ABI of the MI355X (gfx950) quantized matvec/matmul engine.
 *
 * Drop-in for the projection path behind the qw35-server engine-side kernel
 * API.  Conventions follow the reference FFI (qw35-server/src/metal/bridge/Qw35FFI.h:1-4):
 *   - every function reports failure by returning 0 (or NULL) and writing a
 *     NUL-terminated message into the caller-provided `err` buffer; success is 1;
 *   - nothing throws across the ABI; GPU execution is asynchronous on the
 *     caller's stream and device-side faults surface at the next
 *     qw35_hip_sync (as they surface at the next wait in the reference,
 *     Qw35FFI.h:87-88).
 * Pointers marked "device" are HBM addresses (hipMalloc'd or offsets into an
 * uploaded model image).  `stream` is a hipStream_t (NULL = default stream).
 * Calls on one stream are ordered.  The library's objects are its plans and
 * runtimes, single-threaded objects (like MetalRuntime, `Send` but not `Sync`,
 * qw35-server/src/metal/bridge.rs:257), and its tensor stores, immutable
 * and shared per model image under a lock; its only other global state is
 * the per-device array of qw35_hip_output_argmax_noalloc.
 *
 * Weight formats are the reference's raw GGUF tensor bytes (no repacking):
 *   type 100  GF4   8 elems / 4 B   (tools/gguf_custom_types.py:26-30)
 *   type 101  GF2   256 elems / 80 B super-blocks: 16 code words, then their
 *             16 e5m2 scale bytes (qw35-server/src/metal/qw35_gf2.metal:1-17;
 *             qw35-server/src/loader/tensors.rs:124-135)
 *   type   8  q8_0 32 elems / 34 B  (qw35-server/src/loader/tensors.rs:142)
 *   type  12  Q4_K 256 elems / 144 B (qw35-server/src/loader/tensors.rs:146)
 *   type  13  Q5_K 256 elems / 176 B (qw35-server/src/loader/tensors.rs:147;
 *             block qw35_block_q5_k, qw35-server/src/metal/qw35_types.metal:9-15)
 *   type  14  Q6_K 256 elems / 210 B (qw35-server/src/loader/tensors.rs:148;
 *             block qw35_block_q6_k, qw35-server/src/metal/qw35_types.metal:17-22)
 *   type   1  F16  1 elem / 2 B (tensors.rs:137): the prefill matmul's weight
 *             form for the k-quants (see qw35_hip_dequantize_f16); the GEMVs
 *             reject it
 * Shape limits of this build: k % 256 == 0 and 256 <= k <= 65536 (the
 * GEMVs take rows longer than 12288 in rounds of 32 chunks of 256 columns);
 * q8_0, whose blocks are 32 columns, takes any k % 32 == 0 up to 65536 in the
 * decode GEMVs (a row-wise kernel when k % 256 != 0, as the reference's
 * n_blocks = ceil(k / 32), Qw35MetalRuntime+FFN.m:240), while its prefill
 * matmul and greedy head need k % 256 == 0 (every Qwen3.5 projection has
 * it); Q6_K also needs k % 512 == 0 and rows * row bytes
 * a multiple of 16 (its 210-byte super-blocks are read as the 16-byte
 * segments that cover them); rows >= 1; n_batch 1..8; a prefill call takes
 * n_tokens * k <= 2^30.
 */
#ifndef QW35_HIP_H
#define QW35_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QW35_HIP_TYPE_F16 1u
#define QW35_HIP_TYPE_Q8_0 8u
#define QW35_HIP_TYPE_Q4_K 12u
#define QW35_HIP_TYPE_Q5_K 13u
#define QW35_HIP_TYPE_Q6_K 14u
#define QW35_HIP_TYPE_GF4 100u
#define QW35_HIP_TYPE_GF2 101u
#define QW35_HIP_MAX_BATCH 8u
/* Largest prefill chunk of a projection runtime (qw35_hip_runtime_create). */
#define QW35_HIP_MAX_PREFILL_CHUNK 4096u

/* GGUF tensor descriptor; field-for-field the reference's
 * qw35_metal_tensor_desc (qw35-server/src/metal/bridge/Qw35MetalTypes.h:18-27),
 * so the Rust #[repr(C)] mirror in bridge.rs is reused unchanged. */
typedef struct {
    const uint8_t *name;
    uintptr_t name_len;
    uint64_t dims[4]; /* dims[0] = k (columns), dims[1] = rows */
    uint32_t n_dims;
    uint32_t type_id;
    uint64_t abs_offset; /* byte offset of the tensor data in the model image */
    uint64_t bytes;
    uint64_t elements;
} qw35_hip_tensor_desc;

/* A weight matrix resident in device memory (raw GGUF bytes, row-major). */
typedef struct {
    const void *data; /* device, 16-byte aligned */
    uint64_t k;       /* columns = dims[0] */
    uint64_t rows;    /* dims[1] */
    uint64_t bytes;   /* rows * row_bytes(type, k) */
    uint32_t type_id; /* QW35_HIP_TYPE_* */
    uint32_t reserved;
} qw35_hip_weight;

/* GGUF v3 reader over a host image of a model file (e.g. an mmap): the
 * reference loader's parse_mapping (qw35-server/src/loader/tensors.rs:23-121):
 * GGUF magic, version 3 only, metadata walked and skipped
 * (loader/metadata.rs:206-288) except general.alignment (u32; 0 keeps 32),
 * 1..8 dimensions, byte sizes by tensor_nbytes (tensors.rs:123-172) for
 * every GGUF type the reference knows, data section at the aligned end of the
 * tensor infos, every tensor inside the image.  *n_tensors = tensor count;
 * out[0 .. min(cap, count)) are filled as bridge.rs:279-290 fills
 * qw35_metal_tensor_desc (dims padded with 1, n_dims the true count, name
 * pointing into model_map, abs_offset from the image start); out may be NULL
 * with cap 0 to query the count.  *data_offset (nullable) = data section. */
int qw35_hip_gguf_parse(const void *model_map, uint64_t model_size, qw35_hip_tensor_desc *out, uint32_t cap,
                        uint32_t *n_tensors, uint64_t *data_offset, char *err, uintptr_t err_len);

/* Device tensor store: replaces Qw35TensorStore (Qw35TensorStore.m:58-153),
 * which wraps the host mmap in Metal buffers.  HBM is not host memory, so the
 * image's bytes 0 .. end of the last tensor are copied once (synchronously)
 * into one device allocation; descs (e.g. from qw35_hip_gguf_parse) are
 * checked to lie inside model_size and copied with their names, so the host
 * image may be unmapped afterwards.  One store per model image and device is
 * shared, as the reference shares one store per mapped file between its
 * runtimes (Qw35MetalRuntime.m:42-80): a create over the same (model_map,
 * model_size) on the same device with the same descriptors (every field and
 * name equal) returns the existing store with one more reference, and
 * qw35_hip_store_destroy drops one; the device copy is freed with the last.
 * Other descriptors over the same image get a store of their own.  The store is immutable after creation,
 * so its users may be on different threads.  Sharing is keyed by the image's
 * address: an image must not be changed, or freed and replaced at the same
 * address, while a store over it is alive.  qw35_hip_store_weight gives the
 * weight view (as qw35_hip_weight_view) of the tensor named
 * name[0 .. name_len).  Drop the last reference after the last kernel that
 * reads the store has completed. */
void *qw35_hip_store_create(const void *model_map, uint64_t model_size, const qw35_hip_tensor_desc *descs,
                            uint32_t count, char *err, uintptr_t err_len);
const void *qw35_hip_store_device_base(const void *store);
uint64_t qw35_hip_store_bytes(const void *store);
int qw35_hip_store_weight(const void *store, const char *name, uintptr_t name_len, qw35_hip_weight *out, char *err,
                          uintptr_t err_len);
void qw35_hip_store_destroy(void *store);

/* 1 if a HIP device is present.  Replaces qw35_metal_has_device (Qw35FFI.h:18-19). */
int qw35_hip_has_device(void);

/* Validate a GGUF tensor descriptor and build the device view
 * data = device_base + desc->abs_offset.  Replaces the no-copy tensor view
 * creation of Qw35TensorStore (Qw35TensorStore.m:58-153) plus the per-type
 * byte-size rule of tensor_nbytes (qw35-server/src/loader/tensors.rs:123-172). */
int qw35_hip_weight_view(const qw35_hip_tensor_desc *desc, const void *device_base, qw35_hip_weight *out,
                         char *err, uintptr_t err_len);

/* Decode GEMV, batch 1..8:
 *   dst[b][r] (+)= sum_k W[r][k] * awq[k] * x[b][k]    (awq == NULL: 1)
 * x: device fp32 [n_batch][k] (16-byte aligned rows); dst: device fp32
 * [n_batch][rows]; residual != 0 adds into dst.  Replaces
 * encodeDecodeMatvecTensor:weight:input:inputOffset:dst:residual:
 * (qw35-server/src/metal/bridge/Qw35MetalRuntime+FFN.m:184-256); the input
 * offset of the reference is folded into `x`.  awq is the explicit form of
 * the AWQ per-input-channel scale that the reference folds into the norm
 * weight (tools/cook_qw35_awq_gf4.py:112-114). */
int qw35_hip_decode_matvec(const qw35_hip_weight *w, const float *x, const float *awq, float *dst,
                           uint32_t n_batch, int residual, void *stream, char *err, uintptr_t err_len);

/* Fused gate/up GEMV + SwiGLU, batch 1..8:
 *   dst[b][r] = silu(gate[r] . (awq*x[b])) * (up[r] . (awq*x[b])),  silu(v) = v / (1 + exp(-v))
 * gate and up share type and shape.  Replaces encodeGf4FusedFfn
 * (Qw35MetalRuntime+FFN.m:13-35) / qw35_ffn_gate_up_swiglu_gf4_f32
 * (qw35-server/src/metal/qw35_gf4.metal:62-96), for GF4, GF2, q8_0, Q4_K and Q5_K
 * (Q6_K is rejected: the reference uses it for the LM head only). */
int qw35_hip_ffn_gate_up_swiglu(const qw35_hip_weight *gate, const qw35_hip_weight *up, const float *x,
                                const float *awq, float *dst, uint32_t n_batch, void *stream, char *err,
                                uintptr_t err_len);

/* Decode GEMV with a K-split workspace (otherwise qw35_hip_decode_matvec):
 * at batch 3..8 on k = 12288 matrices of at most 4096 rows (the down
 * projection) every workgroup of the plain launch would convert the whole
 * activation batch, so with a workspace the launch splits K four ways across
 * workgroups of four row tiles; each writes its partial sums to the workspace
 * and the last of a
 * row group to finish adds them in a fixed order (so results do not depend
 * on timing) and writes dst.  workspace: device memory of at least
 * qw35_hip_decode_matvec_workspace_size(w, n_batch) bytes (0: this call never
 * splits; a smaller workspace disables the split), 256-byte aligned,
 * zero-filled before its first use; its first 1 KiB holds the row-group
 * counters, which every call returns to zero, so a workspace can be reused
 * by later calls of any shape and by plans on the same stream, but not by
 * calls that overlap.  NULL behaves as qw35_hip_decode_matvec.  No
 * counterpart in the reference, whose decode dispatch allocates per runtime. */
uint64_t qw35_hip_decode_matvec_workspace_size(const qw35_hip_weight *w, uint32_t n_batch);
int qw35_hip_decode_matvec_ws(const qw35_hip_weight *w, const float *x, const float *awq, float *dst,
                              uint32_t n_batch, int residual, void *workspace, uint64_t workspace_bytes, void *stream,
                              char *err, uintptr_t err_len);

/* The kernel a qw35_hip_decode_matvec (w_up NULL) or qw35_hip_ffn_gate_up_swiglu
 * (w_up set) call with this weight, batch and AWQ presence launches -- with a
 * K-split workspace when with_workspace != 0 (as plans and
 * qw35_hip_decode_matvec_ws have) -- named as the profiler names it (e.g.
 * "gf4_mfma_gemv<1, 3, 8, 2, false, false, true>"), with its grid, workgroup
 * size, LDS bytes and K-split workspace bytes (0: no split); nothing is
 * launched.  For a batch the GF4 kernel splits, its first launch.  No
 * counterpart in the reference: it matches measurements and tests to the
 * launch plan. */
int qw35_hip_gemv_kernel(const qw35_hip_weight *w, const qw35_hip_weight *w_up, uint32_t n_batch, int has_awq,
                         int with_workspace, char *name, uintptr_t name_len, uint32_t *grid, uint32_t *block,
                         uint32_t *lds_bytes, uint64_t *workspace_bytes, char *err, uintptr_t err_len);

/* Greedy LM head: per batch row b, the largest of
 *   logit[r] = sum_k W[r][k] * awq[k] * x[b][k]
 * over the rows r, written as token[b] = r (uint32) and logit[b], without
 * materialising the logits; ties go to the smaller row, NaN is never chosen
 * (an all-NaN row gives 0xFFFFFFFF and -inf).  Replaces the greedy path of
 * encodeOutputHead (qw35-server/src/metal/bridge/Qw35MetalRuntime+Output.m:11-65):
 * qw35_output_q6_k_argmax_partials_16row_f32 + qw35_output_argmax_reduce_partials_f32
 * (qw35-server/src/metal/qw35_output.metal:2-182).  Any supported type (the
 * reference's head is Q6_K or GF4).  For the k-quants and GF2 the logits are
 * bit-identical to qw35_hip_decode_matvec's.  Two launches on `stream`;
 * workspace: device memory of qw35_hip_output_argmax_workspace_size(w, n_batch)
 * bytes (256-byte aligned, caller-owned, not shared by concurrent calls). */
uint64_t qw35_hip_output_argmax_workspace_size(const qw35_hip_weight *w, uint32_t n_batch);
int qw35_hip_output_argmax(const qw35_hip_weight *w, const float *x, const float *awq, uint32_t n_batch,
                           uint32_t *token, float *logit, void *workspace, uint64_t workspace_bytes, void *stream,
                           char *err, uintptr_t err_len);

/* Greedy head that allocates nothing and takes no workspace: the same
 * validation, kernels and results (bit for bit) as qw35_hip_output_argmax,
 * with the per-workgroup partials in a device array the library owns,
 * QW35_HIP_ARGMAX_SCRATCH_BYTES on each GPU it runs on, held until the
 * process ends.  No counterpart in the reference: it is for callers that
 * cannot allocate or pass a workspace (code under HIP graph capture, tight
 * serving loops, harnesses that forbid allocation).  A head whose partials
 * exceed the array (2 x 4 x n_batch x the GEMV's workgroup count, each half
 * rounded up to 256 bytes; e.g. every plan of a 248320 x 4096 head at batch
 * 1..8 fits) is refused with an error.  All calls on one GPU share its
 * array, which keeps the last call's partials: calls that overlap on one GPU
 * (concurrent streams, or threads) race and must be serialised by the
 * caller.  The first call on each device looks the array up
 * (hipGetSymbolAddress); make it outside graph capture. */
#define QW35_HIP_ARGMAX_SCRATCH_BYTES (2u << 20)
int qw35_hip_output_argmax_noalloc(const qw35_hip_weight *w, const float *x, const float *awq, uint32_t n_batch,
                                   uint32_t *token, float *logit, void *stream, char *err, uintptr_t err_len);

/* fp32 dequantisation (bit-exact statement of each format).  row_ids == NULL:
 * all rows, dst fp32 [rows][k]; otherwise dst[i] = row row_ids[i] (device
 * uint32 [n_rows]; an id >= rows gives a row of zeros), which is the
 * embedding gather of qw35_get_row(s)_{q8_0,q4_k}_f32
 * (qw35-server/src/metal/qw35_matvec.metal:100-169). */
int qw35_hip_dequantize(const qw35_hip_weight *w, const uint32_t *row_ids, uint32_t n_rows, float *dst,
                        void *stream, char *err, uintptr_t err_len);

/* fp16 prefill image of a weight: dst (device, 16-byte aligned, rows * k
 * halves, row-major) = fp16_rne(dequantised W), the exact value for GF4 and
 * the rounding the reference's tiled matmul applies when it dequantises a
 * k-quant weight tile to half (qw35_kernel_mul_mm, qw35-server/src/metal/
 * qw35_tiled_mm.metal:199-255).  Viewed as a type-1 (F16) weight it is the
 * operand of qw35_hip_matmul_prefill for GF2 / q8_0 / Q4_K / Q5_K / Q6_K projections; made
 * once and kept resident (2 bytes per weight: about 4.2 GB for the 9B's q8_0
 * projections). */
int qw35_hip_dequantize_f16(const qw35_hip_weight *w, void *dst, void *stream, char *err, uintptr_t err_len);

/* Decode-step plan: a fixed sequence of projection GEMVs recorded once into a
 * hipGraph and replayed per token.  Replaces the per-token recording of the
 * projection dispatches in evalToken / encodeDecodeLayers
 * (qw35-server/src/metal/bridge/Qw35MetalRuntime.m:807-880,1170-1221) and
 * encodeGf4FusedFfn (Qw35MetalRuntime+FFN.m:13-35).  Every op reads and writes
 * the device buffers named at create time, so callers refresh the inputs in
 * place between launches.  The weights pointed to by an op are copied into the
 * plan; the device memory they describe must outlive it. */
#define QW35_HIP_OP_MATVEC 0u /* dst (+)= W (awq * x), see qw35_hip_decode_matvec */
#define QW35_HIP_OP_SWIGLU 1u /* dst = silu(gate (awq*x)) * (up (awq*x)) */
#define QW35_HIP_OP_ARGMAX 2u /* greedy head, see qw35_hip_output_argmax: token[b], dst[b] = logit */
/* Multi-token ops (a prefill chunk): the prefill matmul of fp32 activations
 * into fp32 dst, n_batch = the chunk's tokens (1..65536), through the op's
 * workspace (qw35_hip_matmul_prefill_epilogue). */
#define QW35_HIP_OP_MATMUL 3u        /* dst (+)= W (awq * x): STORE, or ADD with residual */
/* dst = silu(gate (awq*x)) * (up (awq*x)): the gate launch (STORE) and the up
 * launch (SWIGLU epilogue), or for GF4 weights one fused launch -- with the
 * same bits where it keeps the gate's planned tile, else (some chunk lengths)
 * within fp32 rounding of them */
#define QW35_HIP_OP_MATMUL_SWIGLU 4u
typedef struct {
    uint32_t kind;               /* QW35_HIP_OP_* */
    uint32_t n_batch;            /* 1..8; MATMUL / MATMUL_SWIGLU: tokens, 1..65536 */
    int32_t residual;            /* MATVEC / MATMUL: nonzero adds into dst */
    uint32_t reserved;
    const qw35_hip_weight *w;    /* MATVEC / MATMUL / ARGMAX weight or SWIGLU / MATMUL_SWIGLU gate */
    const qw35_hip_weight *w_up; /* SWIGLU / MATMUL_SWIGLU up, else NULL */
    const float *x;              /* device [n_batch][k] */
    const float *awq;            /* device [k] or NULL */
    float *dst;                  /* device [n_batch][rows]; ARGMAX: the chosen logits [n_batch] */
    /* ARGMAX only (NULL otherwise): the chosen rows [n_batch]. */
    uint32_t *token;
    /* ARGMAX: a workspace of qw35_hip_output_argmax_workspace_size(w, n_batch)
     * bytes used by this op alone.  MATMUL / MATMUL_SWIGLU: a prefill
     * workspace (qw35_hip_matmul_prefill_workspace_size), which ops that run
     * one after the other may share.  256-byte aligned; NULL / 0 for the
     * other kinds. */
    void *workspace;
    uint64_t workspace_bytes;
} qw35_hip_plan_op;

/* Consecutive ops over the same x, awq and batch may be recorded as one
 * launch: MATVEC ops of a q8_0 / Q4_K / Q6_K type with disjoint outputs, and
 * MATMUL ops of one weight form and k with the same workspace and residual
 * flag, row counts that are multiples of 4 and disjoint outputs (a mixer's
 * input projections); up to 4 ops per launch.  A merged MATMUL launch is
 * planned for the summed rows, so its outputs may differ from the single
 * calls' in the last bits (the K split and the order of the partial sums),
 * not in precision.  Its workspace holds the planned K split when sized by
 * qw35_hip_matmul_prefill_workspace_size of a view with the summed rows and
 * bytes; a smaller one (still at least each op's minimum) splits less.
 *
 * Validate the ops (same rules as the single calls) and record them; NULL on
 * error.  Recording launches nothing.  A plan whose launches split K (see
 * qw35_hip_decode_matvec_ws) allocates and zeroes one workspace for them at
 * creation, freed by qw35_hip_plan_destroy; replays of one plan must not
 * overlap. */
void *qw35_hip_plan_create(const qw35_hip_plan_op *ops, uint32_t n_ops, char *err, uintptr_t err_len);
/* Replay the recorded sequence on `stream` (asynchronous). */
int qw35_hip_plan_launch(void *plan, void *stream, char *err, uintptr_t err_len);
/* Number of ops recorded in the plan (0 for NULL). */
uint32_t qw35_hip_plan_size(const void *plan);
void qw35_hip_plan_destroy(void *plan);

/* ---- Projection runtime: the in-scope part of the runtime-level ABI ----
 *
 * The reference's Rust host drives a whole-model runtime through
 * qw35_metal_runtime_create / eval_token / argmax / copy_logits / sync /
 * destroy (qw35-server/src/metal/bridge/Qw35FFI.h:19-118).  This library
 * builds the part of that runtime that is this path: the model's projection
 * weights resolved by their GGUF names and validated against the
 * hyper-parameters (Qw35MetalRuntime.m:287-372), held in a device tensor store
 * shared by every runtime over the same model image (Qw35MetalRuntime.m:42-80),
 * and one decode step's projections in the reference's dispatch order
 * (encodeDecodeLayers, Qw35MetalRuntime.m:1170-1221) recorded as a hipGraph.
 * The attention, DeltaNet recurrence, norms, embedding and KV cache between
 * the projections are not part of this library: each step reads its inputs
 * from runtime-owned device buffers (qw35_hip_runtime_buffer) that the
 * caller's own kernels fill, as the reference's _norm / _core / _act_a buffers
 * are filled by its non-projection kernels. */

/* Hyper-parameters: field for field the reference's qw35_metal_hparams
 * (Qw35MetalTypes.h:30-59; append-only).  The runtime reads the projection
 * shapes from transformer_layers, embedding_length, feed_forward_length,
 * attention_heads / kv_heads / key_length / value_length, ssm_state_size,
 * ssm_group_count, ssm_time_step_rank, ssm_inner_size,
 * full_attention_interval (0 = 4) and attn_gate; the rest is carried for the
 * caller's kernels.  n_cls_out must be 0 (classification heads are not part
 * of this path). */
typedef struct {
    uint32_t transformer_layers;
    uint32_t embedding_length;
    uint32_t feed_forward_length;
    uint32_t attention_heads;
    uint32_t attention_kv_heads;
    uint32_t attention_key_length;
    uint32_t attention_value_length;
    uint32_t rope_dimension_count;
    int32_t rope_sections[4];
    float rope_freq_base;
    float rms_epsilon;
    uint32_t ssm_conv_kernel;
    uint32_t ssm_state_size;
    uint32_t ssm_group_count;
    uint32_t ssm_time_step_rank;
    uint32_t ssm_inner_size;
    uint32_t full_attention_interval;
    int32_t attn_window;
    int32_t attn_sink;
    uint32_t attn_gate;
    uint32_t n_cls_out;
} qw35_hip_hparams;

/* Output-head mode of an eval call: the reference's qw35_logits_mode
 * (Qw35MetalTypes.h:61-66). */
typedef enum {
    QW35_HIP_LOGITS_NONE = 0,   /* no head */
    QW35_HIP_LOGITS_ARGMAX = 1, /* fused greedy head only; logits never materialised */
    QW35_HIP_LOGITS_FULL = 2,   /* the full logits vector */
} qw35_hip_logits_mode;

/* Runtime-owned fp32 device buffers (the reference runtime's buffers,
 * Qw35MetalRuntime.m:374-460): max(max_batch, prefill_chunk) rows of `width`
 * floats each (the logits: max_batch rows), width being the largest row any
 * op reads or writes there.  Like the reference's max-sized scratch, a
 * buffer holds the n rows of one op packed at that op's own row length: an op
 * of k input columns reads row t at offset t * k, an op of `rows` output rows
 * writes row t at offset t * rows.  So where a buffer serves ops of
 * different lengths (QKV: attn_q and attn_qkv; CORE: attn_output and ssm_out
 * inputs), the row stride of each op is its own length, not `width`. */
#define QW35_HIP_RT_NORM 0u   /* [emb] input of the mixer input projections, the FFN and the head (_norm) */
#define QW35_HIP_RT_CORE 1u   /* input of attn_output [heads*value_length] or ssm_out [ssm_inner] (_core) */
#define QW35_HIP_RT_ACT 2u    /* [emb] residual stream; attn_output, ssm_out and ffn_down add into it (_act_a) */
#define QW35_HIP_RT_QKV 3u    /* output of attn_q [heads*key_length*(attn_gate?2:1)] or attn_qkv
                               * [ssm_inner + 2*groups*state] (_qkv) */
#define QW35_HIP_RT_K 4u      /* [kv_heads*key_length] attn_k output */
#define QW35_HIP_RT_V 5u      /* [kv_heads*value_length] attn_v output */
#define QW35_HIP_RT_Z 6u      /* [ssm_inner] attn_gate output (_z_gate) */
#define QW35_HIP_RT_BETA 7u   /* [ssm_time_step_rank] ssm_beta output (_beta) */
#define QW35_HIP_RT_ALPHA 8u  /* [ssm_time_step_rank] ssm_alpha output (_alpha) */
#define QW35_HIP_RT_FFN 9u    /* [ffn] SwiGLU output, input of ffn_down (_ffn_gate) */
#define QW35_HIP_RT_LOGITS 10u /* [vocab] output head (_logits) */
#define QW35_HIP_RT_NBUF 11u

/* Create a runtime on the current device: parse nothing (descs come from
 * qw35_hip_gguf_parse or the caller's loader), share or create the device
 * store of model_map (qw35_hip_store_create), resolve and validate every
 * projection (blk.N.attn_q/k/v/output or blk.N.attn_qkv/attn_gate/ssm_beta/
 * ssm_alpha/ssm_out by layer kind, blk.N.ffn_gate/up/down, output.weight with
 * vocab_size rows), and allocate the buffers above.  max_batch (1..8): rows
 * of a decode step; prefill_chunk (0..QW35_HIP_MAX_PREFILL_CHUNK): most
 * tokens of a prefill chunk (the reference's prefill_chunk argument of
 * qw35_metal_runtime_create, Qw35FFI.h:37-50; its server's default is 128,
 * its maximum 256, qw35-server/src/model.rs:30-31).  Above 8, the runtime
 * also holds one prefill matmul workspace and, for each projection that is
 * not GF4 or q8_0, its fp16 prefill image (qw35_hip_dequantize_f16: 2 bytes
 * per weight).  NULL on error (missing tensor, shape that does not match
 * hparams, type the GEMVs do not take, gate/up of different types). */
void *qw35_hip_runtime_create(const void *model_map, uint64_t model_size, const qw35_hip_tensor_desc *tensors,
                              uintptr_t tensor_count, const qw35_hip_hparams *hparams, uint32_t vocab_size,
                              uint32_t max_batch, uint32_t prefill_chunk, char *err, uintptr_t err_len);
/* Waits for the runtime's work, then frees it (the store when its last user goes). */
void qw35_hip_runtime_destroy(void *runtime);
/* One decode step's projections for n_batch rows of the buffers, replayed from
 * a hipGraph recorded on first use of (n_batch, logits_mode).  Asynchronous on
 * the runtime's stream: device errors surface at the next sync / argmax /
 * copy_logits, as in the reference (Qw35FFI.h:87-88).  Replaces the projection
 * part of qw35_metal_runtime_eval_token (Qw35FFI.h:92-97). */
int qw35_hip_runtime_eval_step(void *runtime, uint32_t n_batch, int logits_mode, char *err, uintptr_t err_len);
/* One prefill chunk's projections for n_tokens rows of the buffers (1 ..
 * max(max_batch, prefill_chunk)), in evalTokens' order (Qw35MetalRuntime.m:
 * 1227-1333): per layer the mixer input projections over NORM, the mixer
 * output projection over CORE added into ACT, ffn_gate / ffn_up / SwiGLU over
 * NORM into FFN, ffn_down over FFN added into ACT; then the head (logits_mode)
 * on the chunk's last NORM row only, as evalTokens runs encodeOutputHead on
 * the last token.  More than 8 tokens run the prefill matmul with fp32
 * activations (qw35_hip_matmul_prefill_epilogue: ADD for the output
 * projections, SWIGLU for ffn_up), up to 8 the decode GEMVs.  Recorded as a
 * hipGraph on first use of (n_tokens, logits_mode) and replayed; asynchronous
 * like eval_step.  A following argmax / copy_logits reads one row.  Replaces
 * the projection part of qw35_metal_runtime_eval_tokens (Qw35FFI.h:97-105). */
int qw35_hip_runtime_eval_chunk(void *runtime, uint32_t n_tokens, int logits_mode, char *err, uintptr_t err_len);
/* Wait for the last eval; then the greedy head's rows and logits of its n_batch
 * batch rows (that eval must have used QW35_HIP_LOGITS_ARGMAX).  Replaces
 * qw35_metal_runtime_argmax (Qw35FFI.h:106-111). */
int qw35_hip_runtime_argmax(void *runtime, uint32_t *token, float *logit, char *err, uintptr_t err_len);
/* Wait for the last eval (QW35_HIP_LOGITS_FULL) and copy its n_batch x vocab
 * logits into dst (len >= n_batch * vocab floats).  Replaces
 * qw35_metal_runtime_copy_logits (Qw35FFI.h:113-118). */
int qw35_hip_runtime_copy_logits(void *runtime, float *dst, uintptr_t len, char *err, uintptr_t err_len);
/* Wait for all of the runtime's work.  Replaces qw35_metal_runtime_sync (Qw35FFI.h:71-72). */
int qw35_hip_runtime_sync(void *runtime, char *err, uintptr_t err_len);
/* Device address and row width (floats) of buffer `which` (QW35_HIP_RT_*). */
int qw35_hip_runtime_buffer(void *runtime, uint32_t which, float **device_ptr, uint64_t *width, char *err,
                            uintptr_t err_len);
/* The runtime's stream (hipStream_t), for ordering the caller's kernels and copies with its steps. */
void *qw35_hip_runtime_stream(void *runtime);
/* The device tensor store the runtime reads its weights from. */
const void *qw35_hip_runtime_store(void *runtime);

/* Multi-token (prefill) matmul of a GF4, q8_0, Q4_K or F16 weight on MFMA:
 *   c[t][r] = sum_k W[r][k] * v[t][k],  v = awq[k] * a[t][k]   (awq == NULL: v = a)
 * a: device [n_tokens][k], a_dtype QW35_HIP_DTYPE_BF16 or QW35_HIP_DTYPE_F32;
 * c: device [n_tokens][rows], c_dtype QW35_HIP_DTYPE_BF16 (round-to-nearest-
 * even) or QW35_HIP_DTYPE_F32; fp32 accumulation.  Replaces encodeMatvecBatch /
 * encodeTiledKMatmul for type 100 (qw35-server/src/metal/bridge/Qw35MetalRuntime+FFN.m:260-366,
 * kernel qw35_mul_mm_gf4_f32 of qw35_tiled_mm.metal:203-255), for q8_0
 * and Q4_K dequantised in the kernel to the fp16 of their exact values
 * (qw35_mul_mm_q8_0_f32, qw35_mul_mm_q4_k_f32), and, through an F16 weight
 * (the prefill image of qw35_hip_dequantize_f16), for the GF2 / Q5_K / Q6_K
 * projections (qw35_mul_mm_{gf2,q5_k,q6_k}_f32, qw35_tiled_mm.metal:208-254);
 * a q8_0 or Q4_K weight's image gives the same products, at 2 bytes per
 * weight of HBM.
 * 1 <= n_tokens <= 65536, rows <= 2^24; n_tokens * k <= 2^30 for bf16
 * activations, 2^29 for fp32. */
#define QW35_HIP_DTYPE_F32 0u
#define QW35_HIP_DTYPE_BF16 1u
/* workspace: NULL, or device memory of
 * qw35_hip_matmul_prefill_workspace_size(w, n_tokens) bytes (256-byte
 * aligned, owned by the caller, not shared by concurrent calls).
 * With a workspace (the staged path) v is computed in fp32 and staged as
 * fp16 with a per-token power of two 2^e that puts the token's max |v| in
 * [2^14, 2^15), and contracted on fp16 MFMA:
 *   - bf16 activations: fp16_rne(2^e v).  Without AWQ every activation of at
 *     least 2^-28 of its token's largest is carried exactly (smaller ones
 *     round at 2^-39 of the largest); with AWQ the product is rounded once,
 *     to fp16;
 *   - fp32 activations: an fp16 hi/lo pair, hi = fp16_rne(2^e v) and
 *     lo = fp16_rne((2^e v - hi) * 2^11), contracted as hi + 2^-11 lo: about
 *     22 significant bits of every activation, the fp32 activations of the
 *     reference's tiled matmul (qw35_tiled_mm.metal:200-224), at twice the
 *     MFMA work of bf16 input.
 * Shapes with too few output tiles for the device also split K, with fp32
 * partial sums in the workspace reduced in a fixed order.  Without a
 * workspace (GF4 only) the loader converts the activations to bf16 and
 * contracts on bf16 MFMA; that path takes bf16 activations without AWQ only
 * (the operands it represents exactly).  The size depends on the weight's
 * shape and n_tokens and covers both activation types (0: invalid weight or
 * n_tokens); a smaller workspace that still holds the staged activations (2
 * bytes per staged activation, 4 per token, each part rounded up to 256
 * bytes; fp32 activations stage two rows per token in groups of 32 tokens:
 * 64 * ceil(n_tokens / 32) rows) is accepted and splits K less.  F16, q8_0
 * and Q4_K weights always take the staged path (the workspace is required). */
uint64_t qw35_hip_matmul_prefill_workspace_size(const qw35_hip_weight *w, uint32_t n_tokens);
int qw35_hip_matmul_prefill(const qw35_hip_weight *w, const void *a, uint32_t a_dtype, const float *awq, void *c,
                            uint32_t c_dtype, uint32_t n_tokens, void *workspace, uint64_t workspace_bytes,
                            void *stream, char *err, uintptr_t err_len);
/* The prefill matmul with the result r = W v written through an epilogue
 * (fp32 c and a workspace; the other arguments as qw35_hip_matmul_prefill):
 *   QW35_HIP_EPILOGUE_STORE   c = r                (qw35_hip_matmul_prefill)
 *   QW35_HIP_EPILOGUE_ADD     c += r               (the residual add of the decode GEMVs, for
 *                                                   attn_output / ssm_out / ffn_down over a chunk)
 *   QW35_HIP_EPILOGUE_SWIGLU  c = silu(c) * r      (c holds the ffn_gate product, r is ffn_up's:
 *                                                   encodeSwiGLU, Qw35MetalRuntime+FFN.m:369-383,
 *                                                   kernel qw35_swiglu_f32 of qw35_core.metal:149,
 *                                                   fused into the up projection)
 * silu(v) = v / (1 + exp(-v)) (qw35_types.metal:40-42).  With a K split the
 * epilogue is applied once, to the sum of the splits.  The reference runs
 * ffn_gate and ffn_up as two tiled matmuls and SwiGLU as a third dispatch
 * (Qw35MetalRuntime.m:1298-1301); here the third is the up matmul's epilogue. */
/* The matmul kernel a qw35_hip_matmul_prefill(_epilogue) call with this
 * weight, token count, activation and output type and AWQ presence launches
 * -- with a workspace of the planned size when with_workspace != 0 (the
 * staged path; its staging pass, prefill_stage_kernel, and a split's
 * reduction, prefill_split_reduce, run beside it), else the path without
 * one -- named as the profiler names it (e.g.
 * "gf4_prefill_f16_kernel<64, 8, 1, 2, false, false, false, 4>"), with its
 * grid, workgroup size, LDS bytes and K splits; nothing is launched.  No
 * counterpart in the reference: it matches measurements and tests to the
 * launch plan. */
int qw35_hip_prefill_kernel(const qw35_hip_weight *w, uint32_t n_tokens, uint32_t a_dtype, int has_awq,
                            uint32_t c_dtype, int with_workspace, char *name, uintptr_t name_len, uint32_t *grid,
                            uint32_t *block, uint32_t *lds_bytes, uint32_t *splits, char *err, uintptr_t err_len);
#define QW35_HIP_EPILOGUE_STORE 0u
#define QW35_HIP_EPILOGUE_ADD 1u
#define QW35_HIP_EPILOGUE_SWIGLU 2u
int qw35_hip_matmul_prefill_epilogue(const qw35_hip_weight *w, const void *a, uint32_t a_dtype, const float *awq,
                                     void *c, uint32_t c_dtype, uint32_t epilogue, uint32_t n_tokens,
                                     void *workspace, uint64_t workspace_bytes, void *stream, char *err,
                                     uintptr_t err_len);

/* Weight producer: fp32 src [rows][k] (device, 16-byte aligned) -> raw tensor
 * bytes of type_id in dst (device, 16-byte aligned, rows * row_bytes(type, k)
 * bytes).  col_scale (device fp32 [k], 16-byte aligned, nullable) multiplies
 * column c before encoding: the AWQ column scale of pack_ffn_gf4
 * (tools/qw35_cook_common.py:182-199).  GF4 is bit-identical to the reference
 * packer pack_gf4_prepared(rows, scale_search=False) (:83-119).  q8_0 (k % 32),
 * Q4_K, Q5_K, Q6_K and GF2 (k % 256) are this library's min/max encoders; the reference
 * has none (it reads those types through gguf-py).  src must be finite. */
int qw35_hip_quantize(uint32_t type_id, const float *src, uint64_t rows, uint64_t k, const float *col_scale,
                      void *dst, void *stream, char *err, uintptr_t err_len);

/* Streaming-read probe: reads every byte of the device buffer `buf` once
 * (`bytes` a multiple of 16, 16-byte aligned) and writes one XOR digest per
 * workgroup into `sink` (device, qw35_hip_stream_read_sink_len(bytes) uint32
 * values).  No counterpart in the reference: it measures the HBM read ceiling
 * that the GEMV bandwidths are reported against. */
uint32_t qw35_hip_stream_read_sink_len(uint64_t bytes);
int qw35_hip_stream_read(const void *buf, uint64_t bytes, uint32_t *sink, void *stream, char *err,
                         uintptr_t err_len);

/* MFMA throughput probe: n_workgroups x 4 waves each run `iters` rounds of 8
 * independent v_mfma_f32_32x32x16_f16 (the prefill kernel's instruction;
 * 32768 flops each) with no memory traffic, so a timed call measures the
 * sustained fp16 MFMA rate (flops = n_workgroups * iters * 1048576).  sink:
 * device fp32 [n_workgroups * 256].  No counterpart in the reference: it
 * measures the ceiling the prefill utilisation is reported against. */
int qw35_hip_mfma_probe(uint32_t n_workgroups, uint32_t iters, float *sink, void *stream, char *err,
                        uintptr_t err_len);

/* Wait for the stream and report any asynchronous device error.  Replaces
 * qw35_metal_runtime_sync (Qw35FFI.h:71-72). */
int qw35_hip_sync(void *stream, char *err, uintptr_t err_len);

#ifdef __cplusplus
}
#endif

#endif /* QW35_HIP_H */
