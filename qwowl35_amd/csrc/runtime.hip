// Projection runtime: the in-scope part of the reference's runtime-level ABI
// (qw35-server/src/metal/bridge/Qw35FFI.h:19-118, Qw35FFI.m).
//
//   * create: the device tensor store shared per model image (as
//     qw35_shared_tensor_store, Qw35MetalRuntime.m:42-80), every projection
//     resolved by its GGUF name and checked against the hyper-parameters (as
//     resolveLayerTensors, Qw35MetalRuntime.m:287-372, and the attn_q row check
//     there), and the activation buffers sized as allocateBuffers does
//     (Qw35MetalRuntime.m:374-460);
//   * eval_step: one decode step's projections in encodeDecodeLayers' order
//     (Qw35MetalRuntime.m:1170-1221: mixer input projections over the layer
//     norm, the mixer output projection added into the residual stream, the
//     fused gate/up/SwiGLU and the down projection added into the residual
//     stream; then the head of encodeOutputHead, +Output.m:11-65), recorded
//     once per (batch, logits mode) as a decode plan (hipGraph) and replayed;
//   * eval_chunk: the projections of one prefill chunk in evalTokens' order
//     (Qw35MetalRuntime.m:1227-1333: per layer the mixer input projections,
//     the mixer output projection, ffn_gate / ffn_up / SwiGLU and ffn_down
//     over the chunk's tokens through encodeMatvecBatch, +FFN.m:260-306; the
//     head on the chunk's last token), recorded once per (tokens, logits
//     mode).  Chunks of more than 8 tokens run the prefill matmul with fp32
//     activations, the output projections adding into the residual stream and
//     the up projection applying SwiGLU in its epilogue; up to 8 tokens run
//     the decode GEMVs;
//   * argmax / copy_logits / sync: wait for the last step and read back, as
//     readArgmaxToken / copyLogits (+Output.m:71-92).
// The runtime owns one non-blocking stream at default priority; it is a
// single-threaded object like MetalRuntime (Send, not Sync, bridge.rs:257).
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <new>
#include <utility>
#include <vector>

#include "../../include/qw35_hip.h"
#include "qw35_kernels.h"

namespace {

void rt_err(char* err, uintptr_t err_len, const char* fmt, ...) {
    if (!err || err_len == 0) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, (size_t)err_len, fmt, ap);
    va_end(ap);
}

bool rt_hip(hipError_t e, const char* what, char* err, uintptr_t err_len) {
    if (e == hipSuccess) return true;
    rt_err(err, err_len, "%s: %s", what, hipGetErrorString(e));
    return false;
}

// Makes the runtime's device current for the scope of an entry point.
struct DeviceScope {
    int prev = -1;
    bool ok = false;
    explicit DeviceScope(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) return;
        ok = prev == dev || hipSetDevice(dev) == hipSuccess;
    }
    ~DeviceScope() {
        if (ok && prev >= 0) (void)hipSetDevice(prev);
    }
};

struct MixProj {
    qw35_hip_weight w;
    qw35_hip_weight pf;  // the weight the prefill matmul takes (w, or its fp16 image)
    uint32_t out;        // QW35_HIP_RT_* buffer it writes
};

struct Layer {
    bool attention = false;
    std::vector<MixProj> mix;  // attention: q, k, v; delta: qkv, gate, beta, alpha
    qw35_hip_weight out{};      // attn_output / ssm_out
    qw35_hip_weight gate{}, up{}, down{};
    qw35_hip_weight out_pf{}, gate_pf{}, up_pf{}, down_pf{};  // prefill forms
};

struct Runtime {
    int device = -1;
    hipStream_t stream = nullptr;
    void* store = nullptr;
    qw35_hip_hparams h{};
    uint32_t vocab = 0, max_batch = 0;
    uint32_t chunk = 0;     // most tokens of a prefill chunk (0: decode batches only)
    uint32_t rows_cap = 0;  // rows of the activation buffers: max(max_batch, chunk)
    std::vector<Layer> layers;
    qw35_hip_weight head{};
    float* buf[QW35_HIP_RT_NBUF] = {};
    uint64_t width[QW35_HIP_RT_NBUF] = {};
    uint32_t* token = nullptr;  // [max_batch] greedy-head rows
    float* logit = nullptr;     // [max_batch] greedy-head logits
    void* am_ws = nullptr;      // greedy-head partials
    uint64_t am_ws_bytes = 0;
    std::map<std::pair<uint32_t, int>, void*> plans;        // (n_batch, logits mode) -> decode plan
    std::map<std::pair<uint32_t, int>, void*> chunk_plans;  // (tokens, logits mode) -> prefill chunk plan
    std::vector<void*> images;  // fp16 prefill images of the k-quant projections
    void* pf_ws = nullptr;      // prefill matmul workspace, shared by a chunk's launches
    uint64_t pf_ws_bytes = 0;
    uint32_t last_batch = 0;
    int last_mode = -1;
};

void runtime_free(Runtime* r) {
    if (!r) return;
    DeviceScope dev(r->device);
    if (r->stream) (void)hipStreamSynchronize(r->stream);
    for (auto& kv : r->plans) qw35_hip_plan_destroy(kv.second);
    for (auto& kv : r->chunk_plans) qw35_hip_plan_destroy(kv.second);
    for (void* p : r->images) (void)hipFree(p);
    if (r->pf_ws) (void)hipFree(r->pf_ws);
    for (float* p : r->buf)
        if (p) (void)hipFree(p);
    if (r->token) (void)hipFree(r->token);
    if (r->logit) (void)hipFree(r->logit);
    if (r->am_ws) (void)hipFree(r->am_ws);
    if (r->store) qw35_hip_store_destroy(r->store);
    if (r->stream) (void)hipStreamDestroy(r->stream);
    delete r;
}

bool gemv_type(uint32_t t) {
    return t == QW35_HIP_TYPE_GF4 || t == QW35_HIP_TYPE_GF2 || t == QW35_HIP_TYPE_Q8_0 || t == QW35_HIP_TYPE_Q4_K ||
           t == QW35_HIP_TYPE_Q5_K || t == QW35_HIP_TYPE_Q6_K;
}

// blk.<il>.<suffix>.weight (or the bare name for il < 0) of the expected shape.
bool resolve(Runtime* r, int il, const char* suffix, uint64_t rows, uint64_t k, qw35_hip_weight* out, char* err,
             uintptr_t err_len) {
    char name[96];
    if (il >= 0)
        snprintf(name, sizeof name, "blk.%d.%s.weight", il, suffix);
    else
        snprintf(name, sizeof name, "%s", suffix);
    char why[256];
    if (!qw35_hip_store_weight(r->store, name, strlen(name), out, why, sizeof why)) {
        rt_err(err, err_len, "runtime_create: %s: %s", name, why);
        return false;
    }
    if (!gemv_type(out->type_id)) {
        rt_err(err, err_len, "runtime_create: %s has type %u, which the decode GEMVs do not take", name, out->type_id);
        return false;
    }
    if (out->rows != rows || out->k != k) {
        rt_err(err, err_len, "runtime_create: %s is %llu x %llu (rows x k), expected %llu x %llu from the hparams",
               name, (unsigned long long)out->rows, (unsigned long long)out->k, (unsigned long long)rows,
               (unsigned long long)k);
        return false;
    }
    return true;
}

bool check_hparams(const qw35_hip_hparams& h, uint32_t vocab, uint32_t max_batch, uint32_t chunk, char* err,
                   uintptr_t err_len) {
    if (h.transformer_layers == 0 || h.transformer_layers > 4096 || h.embedding_length == 0 ||
        h.feed_forward_length == 0) {
        rt_err(err, err_len, "runtime_create: transformer_layers, embedding_length and feed_forward_length must be "
                             "positive");
        return false;
    }
    if (h.n_cls_out != 0) {
        rt_err(err, err_len, "runtime_create: classification heads (n_cls_out=%u) are not part of this runtime",
               h.n_cls_out);
        return false;
    }
    if (vocab == 0) {
        rt_err(err, err_len, "runtime_create: vocab_size must be positive");
        return false;
    }
    if (max_batch < 1 || max_batch > QW35_HIP_MAX_BATCH) {
        rt_err(err, err_len, "runtime_create: max_batch=%u must be in 1..%u", max_batch, QW35_HIP_MAX_BATCH);
        return false;
    }
    if (chunk > QW35_HIP_MAX_PREFILL_CHUNK) {
        rt_err(err, err_len, "runtime_create: prefill_chunk=%u must be in 0..%u", chunk, QW35_HIP_MAX_PREFILL_CHUNK);
        return false;
    }
    return true;
}

bool is_attention(const qw35_hip_hparams& h, uint32_t il) {
    const uint32_t interval = h.full_attention_interval ? h.full_attention_interval : 4;
    return ((il + 1) % interval) == 0;
}

// The decode-step ops for n_batch rows and a logits mode, in dispatch order.
std::vector<qw35_hip_plan_op> step_ops(const Runtime& r, uint32_t nb, int mode) {
    std::vector<qw35_hip_plan_op> ops;
    auto op = [&](uint32_t kind, const qw35_hip_weight* w, const qw35_hip_weight* up, uint32_t in, float* dst,
                  int residual) {
        qw35_hip_plan_op o{};
        o.kind = kind;
        o.n_batch = nb;
        o.residual = residual;
        o.w = w;
        o.w_up = up;
        o.x = r.buf[in];
        o.dst = dst;
        ops.push_back(o);
    };
    for (const Layer& l : r.layers) {
        for (const MixProj& m : l.mix) op(QW35_HIP_OP_MATVEC, &m.w, nullptr, QW35_HIP_RT_NORM, r.buf[m.out], 0);
        op(QW35_HIP_OP_MATVEC, &l.out, nullptr, QW35_HIP_RT_CORE, r.buf[QW35_HIP_RT_ACT], 1);
        op(QW35_HIP_OP_SWIGLU, &l.gate, &l.up, QW35_HIP_RT_NORM, r.buf[QW35_HIP_RT_FFN], 0);
        op(QW35_HIP_OP_MATVEC, &l.down, nullptr, QW35_HIP_RT_FFN, r.buf[QW35_HIP_RT_ACT], 1);
    }
    if (mode == QW35_HIP_LOGITS_FULL) {
        op(QW35_HIP_OP_MATVEC, &r.head, nullptr, QW35_HIP_RT_NORM, r.buf[QW35_HIP_RT_LOGITS], 0);
    } else if (mode == QW35_HIP_LOGITS_ARGMAX) {
        op(QW35_HIP_OP_ARGMAX, &r.head, nullptr, QW35_HIP_RT_NORM, r.logit, 0);
        ops.back().token = r.token;
        ops.back().workspace = r.am_ws;
        ops.back().workspace_bytes = r.am_ws_bytes;
    }
    return ops;
}

// The head on the chunk's last token: one row of NORM.
void head_op(const Runtime& r, std::vector<qw35_hip_plan_op>& ops, const float* x, int mode) {
    qw35_hip_plan_op o{};
    o.n_batch = 1;
    o.w = &r.head;
    o.x = x;
    if (mode == QW35_HIP_LOGITS_FULL) {
        o.kind = QW35_HIP_OP_MATVEC;
        o.dst = r.buf[QW35_HIP_RT_LOGITS];
        ops.push_back(o);
    } else if (mode == QW35_HIP_LOGITS_ARGMAX) {
        o.kind = QW35_HIP_OP_ARGMAX;
        o.dst = r.logit;
        o.token = r.token;
        o.workspace = r.am_ws;
        o.workspace_bytes = r.am_ws_bytes;
        ops.push_back(o);
    }
}

// A prefill chunk's ops for n tokens, in evalTokens' order: more than 8 tokens
// on the prefill matmul (fp32 activations), else on the decode GEMVs.
std::vector<qw35_hip_plan_op> chunk_ops(const Runtime& r, uint32_t n, int mode) {
    std::vector<qw35_hip_plan_op> ops;
    if (n <= QW35_HIP_MAX_BATCH) {
        ops = step_ops(r, n, QW35_HIP_LOGITS_NONE);
    } else {
        auto op = [&](uint32_t kind, const qw35_hip_weight* w, const qw35_hip_weight* up, uint32_t in, uint32_t out,
                      int residual) {
            qw35_hip_plan_op o{};
            o.kind = kind;
            o.n_batch = n;
            o.residual = residual;
            o.w = w;
            o.w_up = up;
            o.x = r.buf[in];
            o.dst = r.buf[out];
            o.workspace = r.pf_ws;
            o.workspace_bytes = r.pf_ws_bytes;
            ops.push_back(o);
        };
        for (const Layer& l : r.layers) {
            for (const MixProj& m : l.mix) op(QW35_HIP_OP_MATMUL, &m.pf, nullptr, QW35_HIP_RT_NORM, m.out, 0);
            op(QW35_HIP_OP_MATMUL, &l.out_pf, nullptr, QW35_HIP_RT_CORE, QW35_HIP_RT_ACT, 1);
            op(QW35_HIP_OP_MATMUL_SWIGLU, &l.gate_pf, &l.up_pf, QW35_HIP_RT_NORM, QW35_HIP_RT_FFN, 0);
            op(QW35_HIP_OP_MATMUL, &l.down_pf, nullptr, QW35_HIP_RT_FFN, QW35_HIP_RT_ACT, 1);
        }
    }
    head_op(r, ops, r.buf[QW35_HIP_RT_NORM] + (size_t)(n - 1) * r.h.embedding_length, mode);
    return ops;
}

// The prefill matmul's weight for w: w itself (GF4, q8_0, Q4_K), else its
// fp16 image, made on the runtime's stream and owned by the runtime.
bool prefill_form(Runtime* r, const qw35_hip_weight& w, qw35_hip_weight* pf, char* err, uintptr_t err_len) {
    if (w.type_id == QW35_HIP_TYPE_GF4 || w.type_id == QW35_HIP_TYPE_Q8_0 || w.type_id == QW35_HIP_TYPE_Q4_K) {
        *pf = w;
        return true;
    }
    void* img = nullptr;
    if (!rt_hip(hipMalloc(&img, (size_t)w.rows * w.k * 2), "runtime_create: prefill image", err, err_len))
        return false;
    try {
        r->images.push_back(img);
    } catch (...) {
        (void)hipFree(img);
        rt_err(err, err_len, "runtime_create: out of host memory");
        return false;
    }
    if (!qw35_hip_dequantize_f16(&w, img, r->stream, err, err_len)) return false;
    *pf = w;
    pf->type_id = QW35_HIP_TYPE_F16;
    pf->data = img;
    pf->bytes = w.rows * w.k * 2;
    return true;
}

bool wait(Runtime* r, const char* what, char* err, uintptr_t err_len) {
    hipError_t e = hipStreamSynchronize(r->stream);
    if (e == hipSuccess) e = hipGetLastError();
    return rt_hip(e, what, err, err_len);
}

}  // namespace

extern "C" {

void* qw35_hip_runtime_create(const void* model_map, uint64_t model_size, const qw35_hip_tensor_desc* tensors,
                              uintptr_t tensor_count, const qw35_hip_hparams* hparams, uint32_t vocab_size,
                              uint32_t max_batch, uint32_t prefill_chunk, char* err, uintptr_t err_len) {
    if (!model_map || !model_size || !tensors || !tensor_count || !hparams) {
        rt_err(err, err_len, "runtime_create: invalid runtime creation inputs");
        return nullptr;
    }
    if (tensor_count > 0xffffffffu) {
        rt_err(err, err_len, "runtime_create: too many tensors");
        return nullptr;
    }
    const qw35_hip_hparams& h = *hparams;
    if (!check_hparams(h, vocab_size, max_batch, prefill_chunk, err, err_len)) return nullptr;
    Runtime* r = new (std::nothrow) Runtime();
    if (!r) {
        rt_err(err, err_len, "runtime_create: out of host memory");
        return nullptr;
    }
    r->h = h;
    r->vocab = vocab_size;
    r->max_batch = max_batch;
    r->chunk = prefill_chunk;
    r->rows_cap = std::max(max_batch, prefill_chunk);
    if (!rt_hip(hipGetDevice(&r->device), "runtime_create: device", err, err_len) ||
        !rt_hip(hipStreamCreateWithFlags(&r->stream, hipStreamNonBlocking), "runtime_create: stream", err, err_len)) {
        runtime_free(r);
        return nullptr;
    }
    r->store = qw35_hip_store_create(model_map, model_size, tensors, (uint32_t)tensor_count, err, err_len);
    if (!r->store) {
        runtime_free(r);
        return nullptr;
    }

    // Shapes (Qw35MetalRuntime.m:345-351,377-387).
    const uint64_t emb = h.embedding_length, ffn = h.feed_forward_length;
    const uint64_t q_rows = (uint64_t)h.attention_heads * h.attention_key_length * (h.attn_gate ? 2u : 1u);
    const uint64_t k_rows = (uint64_t)h.attention_kv_heads * h.attention_key_length;
    const uint64_t v_rows = (uint64_t)h.attention_kv_heads * h.attention_value_length;
    const uint64_t attn_out_k = (uint64_t)h.attention_heads * h.attention_value_length;
    const uint64_t inner = h.ssm_inner_size;
    const uint64_t qkv_rows = inner + 2ull * h.ssm_group_count * h.ssm_state_size;
    const uint64_t tsr = h.ssm_time_step_rank;
    bool any_attn = false, any_delta = false;
    try {
        r->layers.resize(h.transformer_layers);
        for (uint32_t il = 0; il < h.transformer_layers; ++il) {
            Layer& l = r->layers[il];
            l.attention = is_attention(h, il);
            struct Want {
                const char* suffix;
                uint64_t rows;
                uint32_t out;
            };
            std::vector<Want> mix;
            if (l.attention) {
                any_attn = true;
                mix = {{"attn_q", q_rows, QW35_HIP_RT_QKV}, {"attn_k", k_rows, QW35_HIP_RT_K},
                       {"attn_v", v_rows, QW35_HIP_RT_V}};
            } else {
                any_delta = true;
                mix = {{"attn_qkv", qkv_rows, QW35_HIP_RT_QKV}, {"attn_gate", inner, QW35_HIP_RT_Z},
                       {"ssm_beta", tsr, QW35_HIP_RT_BETA}, {"ssm_alpha", tsr, QW35_HIP_RT_ALPHA}};
            }
            for (const Want& m : mix) {
                MixProj p{};
                p.out = m.out;
                if (!resolve(r, (int)il, m.suffix, m.rows, emb, &p.w, err, err_len)) {
                    runtime_free(r);
                    return nullptr;
                }
                l.mix.push_back(p);
            }
            if (!resolve(r, (int)il, l.attention ? "attn_output" : "ssm_out", emb, l.attention ? attn_out_k : inner,
                         &l.out, err, err_len) ||
                !resolve(r, (int)il, "ffn_gate", ffn, emb, &l.gate, err, err_len) ||
                !resolve(r, (int)il, "ffn_up", ffn, emb, &l.up, err, err_len) ||
                !resolve(r, (int)il, "ffn_down", emb, ffn, &l.down, err, err_len)) {
                runtime_free(r);
                return nullptr;
            }
            if (l.gate.type_id != l.up.type_id || l.gate.type_id == QW35_HIP_TYPE_Q6_K) {
                rt_err(err, err_len,
                       "runtime_create: blk.%u.ffn_gate / ffn_up (types %u, %u) must share a type with a fused "
                       "gate/up form (not q6_k)",
                       il, l.gate.type_id, l.up.type_id);
                runtime_free(r);
                return nullptr;
            }
        }
    } catch (...) {
        rt_err(err, err_len, "runtime_create: out of host memory");
        runtime_free(r);
        return nullptr;
    }
    if (!resolve(r, -1, "output.weight", vocab_size, emb, &r->head, err, err_len)) {
        runtime_free(r);
        return nullptr;
    }

    // Prefill forms and the workspace of chunks of more than 8 tokens: the
    // largest any projection's planned launch uses at any chunk length.
    if (prefill_chunk > QW35_HIP_MAX_BATCH) {
        std::vector<const qw35_hip_weight*> pfs;
        try {
            for (Layer& l : r->layers) {
                for (MixProj& m : l.mix) {
                    if (!prefill_form(r, m.w, &m.pf, err, err_len)) {
                        runtime_free(r);
                        return nullptr;
                    }
                    pfs.push_back(&m.pf);
                }
                if (!prefill_form(r, l.out, &l.out_pf, err, err_len) ||
                    !prefill_form(r, l.gate, &l.gate_pf, err, err_len) ||
                    !prefill_form(r, l.up, &l.up_pf, err, err_len) ||
                    !prefill_form(r, l.down, &l.down_pf, err, err_len)) {
                    runtime_free(r);
                    return nullptr;
                }
                pfs.insert(pfs.end(), {&l.out_pf, &l.gate_pf, &l.down_pf});
            }
        } catch (...) {
            rt_err(err, err_len, "runtime_create: out of host memory");
            runtime_free(r);
            return nullptr;
        }
        std::vector<std::pair<uint32_t, std::pair<uint64_t, uint64_t>>> shapes;  // distinct (type, rows, k)
        for (const qw35_hip_weight* w : pfs) {
            const auto key = std::make_pair(w->type_id, std::make_pair(w->rows, w->k));
            if (std::find(shapes.begin(), shapes.end(), key) != shapes.end()) continue;
            shapes.push_back(key);
            for (uint32_t n = QW35_HIP_MAX_BATCH + 1; n <= prefill_chunk; ++n) {
                const uint64_t b = qw35_hip_matmul_prefill_workspace_size(w, n);
                if (b == 0) {
                    rt_err(err, err_len, "runtime_create: a %llu x %llu projection of type %u has no prefill form",
                           (unsigned long long)w->rows, (unsigned long long)w->k, w->type_id);
                    runtime_free(r);
                    return nullptr;
                }
                r->pf_ws_bytes = std::max(r->pf_ws_bytes, b);
            }
        }
        // A layer's mixer input projections of one weight form and k run as one
        // launch over their summed rows (the plan's segment launches): size that
        // launch too.
        for (const Layer& l : r->layers) {
            for (size_t i = 0; i < l.mix.size();) {
                qw35_hip_weight merged = l.mix[i].pf;
                size_t j = i + 1;
                while (j < l.mix.size() && j - i < (size_t)qw35::kMaxSegments && merged.rows % 4 == 0 &&
                       l.mix[j].pf.type_id == merged.type_id && l.mix[j].pf.k == merged.k &&
                       l.mix[j].pf.rows % 4 == 0)
                    merged.rows += l.mix[j].pf.rows, merged.bytes += l.mix[j++].pf.bytes;
                if (j - i > 1)
                    for (uint32_t n = QW35_HIP_MAX_BATCH + 1; n <= prefill_chunk; ++n)
                        r->pf_ws_bytes = std::max(r->pf_ws_bytes, qw35_hip_matmul_prefill_workspace_size(&merged, n));
                i = j;
            }
        }
        if (!rt_hip(hipMalloc(&r->pf_ws, r->pf_ws_bytes), "runtime_create: prefill workspace", err, err_len) ||
            !rt_hip(hipStreamSynchronize(r->stream), "runtime_create: prefill images", err, err_len)) {
            runtime_free(r);
            return nullptr;
        }
    }

    // Buffers: rows_cap rows of fp32, zeroed (the logits: max_batch rows).
    r->width[QW35_HIP_RT_NORM] = emb;
    r->width[QW35_HIP_RT_CORE] = std::max(any_attn ? attn_out_k : 0, any_delta ? inner : 0);
    r->width[QW35_HIP_RT_ACT] = emb;
    r->width[QW35_HIP_RT_QKV] = std::max(any_attn ? q_rows : 0, any_delta ? qkv_rows : 0);
    r->width[QW35_HIP_RT_K] = any_attn ? k_rows : 0;
    r->width[QW35_HIP_RT_V] = any_attn ? v_rows : 0;
    r->width[QW35_HIP_RT_Z] = any_delta ? inner : 0;
    r->width[QW35_HIP_RT_BETA] = any_delta ? tsr : 0;
    r->width[QW35_HIP_RT_ALPHA] = any_delta ? tsr : 0;
    r->width[QW35_HIP_RT_FFN] = ffn;
    r->width[QW35_HIP_RT_LOGITS] = vocab_size;
    for (uint32_t b = 0; b < QW35_HIP_RT_NBUF; ++b) {
        if (!r->width[b]) continue;
        const size_t rows = b == QW35_HIP_RT_LOGITS ? max_batch : r->rows_cap;
        const size_t bytes = rows * r->width[b] * sizeof(float);
        if (!rt_hip(hipMalloc(&r->buf[b], bytes), "runtime_create: buffer", err, err_len) ||
            !rt_hip(hipMemset(r->buf[b], 0, bytes), "runtime_create: buffer", err, err_len)) {
            runtime_free(r);
            return nullptr;
        }
    }
    for (uint32_t nb = 1; nb <= max_batch; ++nb)
        r->am_ws_bytes = std::max(r->am_ws_bytes, qw35_hip_output_argmax_workspace_size(&r->head, nb));
    if (!rt_hip(hipMalloc(&r->token, max_batch * sizeof(uint32_t)), "runtime_create: head", err, err_len) ||
        !rt_hip(hipMalloc(&r->logit, max_batch * sizeof(float)), "runtime_create: head", err, err_len) ||
        !rt_hip(hipMalloc(&r->am_ws, r->am_ws_bytes), "runtime_create: head workspace", err, err_len) ||
        !rt_hip(hipDeviceSynchronize(), "runtime_create: buffers", err, err_len)) {
        runtime_free(r);
        return nullptr;
    }
    return r;
}

void qw35_hip_runtime_destroy(void* runtime) { runtime_free(static_cast<Runtime*>(runtime)); }

int qw35_hip_runtime_eval_step(void* runtime, uint32_t n_batch, int logits_mode, char* err, uintptr_t err_len) {
    Runtime* r = static_cast<Runtime*>(runtime);
    if (!r) {
        rt_err(err, err_len, "runtime_eval_step: invalid runtime");
        return 0;
    }
    if (n_batch < 1 || n_batch > r->max_batch) {
        rt_err(err, err_len, "runtime_eval_step: n_batch=%u must be in 1..%u", n_batch, r->max_batch);
        return 0;
    }
    if (logits_mode != QW35_HIP_LOGITS_NONE && logits_mode != QW35_HIP_LOGITS_ARGMAX &&
        logits_mode != QW35_HIP_LOGITS_FULL) {
        rt_err(err, err_len, "runtime_eval_step: unknown logits mode %d", logits_mode);
        return 0;
    }
    DeviceScope dev(r->device);
    if (!dev.ok) {
        rt_err(err, err_len, "runtime_eval_step: cannot make device %d current", r->device);
        return 0;
    }
    const auto key = std::make_pair(n_batch, logits_mode);
    auto it = r->plans.find(key);
    void* plan = it == r->plans.end() ? nullptr : it->second;
    if (!plan) {
        std::vector<qw35_hip_plan_op> ops;
        try {
            ops = step_ops(*r, n_batch, logits_mode);
        } catch (...) {
            rt_err(err, err_len, "runtime_eval_step: out of host memory");
            return 0;
        }
        plan = qw35_hip_plan_create(ops.data(), (uint32_t)ops.size(), err, err_len);
        if (!plan) return 0;
        try {
            r->plans[key] = plan;
        } catch (...) {
            qw35_hip_plan_destroy(plan);
            rt_err(err, err_len, "runtime_eval_step: out of host memory");
            return 0;
        }
    }
    if (!qw35_hip_plan_launch(plan, r->stream, err, err_len)) return 0;
    r->last_batch = n_batch;
    r->last_mode = logits_mode;
    return 1;
}

int qw35_hip_runtime_eval_chunk(void* runtime, uint32_t n_tokens, int logits_mode, char* err, uintptr_t err_len) {
    Runtime* r = static_cast<Runtime*>(runtime);
    if (!r) {
        rt_err(err, err_len, "runtime_eval_chunk: invalid runtime");
        return 0;
    }
    if (n_tokens < 1 || n_tokens > r->rows_cap) {
        rt_err(err, err_len, "runtime_eval_chunk: n_tokens=%u must be in 1..%u (max(max_batch, prefill_chunk))",
               n_tokens, r->rows_cap);
        return 0;
    }
    if (logits_mode != QW35_HIP_LOGITS_NONE && logits_mode != QW35_HIP_LOGITS_ARGMAX &&
        logits_mode != QW35_HIP_LOGITS_FULL) {
        rt_err(err, err_len, "runtime_eval_chunk: unknown logits mode %d", logits_mode);
        return 0;
    }
    DeviceScope dev(r->device);
    if (!dev.ok) {
        rt_err(err, err_len, "runtime_eval_chunk: cannot make device %d current", r->device);
        return 0;
    }
    const auto key = std::make_pair(n_tokens, logits_mode);
    auto it = r->chunk_plans.find(key);
    void* plan = it == r->chunk_plans.end() ? nullptr : it->second;
    if (!plan) {
        std::vector<qw35_hip_plan_op> ops;
        try {
            ops = chunk_ops(*r, n_tokens, logits_mode);
        } catch (...) {
            rt_err(err, err_len, "runtime_eval_chunk: out of host memory");
            return 0;
        }
        plan = qw35_hip_plan_create(ops.data(), (uint32_t)ops.size(), err, err_len);
        if (!plan) return 0;
        try {
            r->chunk_plans[key] = plan;
        } catch (...) {
            qw35_hip_plan_destroy(plan);
            rt_err(err, err_len, "runtime_eval_chunk: out of host memory");
            return 0;
        }
    }
    if (!qw35_hip_plan_launch(plan, r->stream, err, err_len)) return 0;
    r->last_batch = 1;  // the head ran on the chunk's last token
    r->last_mode = logits_mode;
    return 1;
}

int qw35_hip_runtime_argmax(void* runtime, uint32_t* token, float* logit, char* err, uintptr_t err_len) {
    Runtime* r = static_cast<Runtime*>(runtime);
    if (!r || !token || !logit) {
        rt_err(err, err_len, "runtime_argmax: invalid runtime or output pointers");
        return 0;
    }
    if (r->last_mode != QW35_HIP_LOGITS_ARGMAX) {
        rt_err(err, err_len, "runtime_argmax: the last eval did not run the greedy head (QW35_HIP_LOGITS_ARGMAX)");
        return 0;
    }
    DeviceScope dev(r->device);
    if (!wait(r, "runtime_argmax", err, err_len)) return 0;
    return rt_hip(hipMemcpy(token, r->token, r->last_batch * sizeof(uint32_t), hipMemcpyDeviceToHost),
                  "runtime_argmax", err, err_len) &&
                   rt_hip(hipMemcpy(logit, r->logit, r->last_batch * sizeof(float), hipMemcpyDeviceToHost),
                          "runtime_argmax", err, err_len)
               ? 1
               : 0;
}

int qw35_hip_runtime_copy_logits(void* runtime, float* dst, uintptr_t len, char* err, uintptr_t err_len) {
    Runtime* r = static_cast<Runtime*>(runtime);
    if (!r) {
        rt_err(err, err_len, "runtime_copy_logits: invalid runtime");
        return 0;
    }
    if (r->last_mode != QW35_HIP_LOGITS_FULL) {
        rt_err(err, err_len, "runtime_copy_logits: the last eval did not compute the logits (QW35_HIP_LOGITS_FULL)");
        return 0;
    }
    const uint64_t n = (uint64_t)r->last_batch * r->vocab;
    if (!dst || len < n) {
        rt_err(err, err_len, "runtime_copy_logits: invalid logits readback buffer (%llu floats needed)",
               (unsigned long long)n);
        return 0;
    }
    DeviceScope dev(r->device);
    if (!wait(r, "runtime_copy_logits", err, err_len)) return 0;
    return rt_hip(hipMemcpy(dst, r->buf[QW35_HIP_RT_LOGITS], n * sizeof(float), hipMemcpyDeviceToHost),
                  "runtime_copy_logits", err, err_len)
               ? 1
               : 0;
}

int qw35_hip_runtime_sync(void* runtime, char* err, uintptr_t err_len) {
    Runtime* r = static_cast<Runtime*>(runtime);
    if (!r) {
        rt_err(err, err_len, "runtime_sync: invalid runtime");
        return 0;
    }
    DeviceScope dev(r->device);
    return wait(r, "runtime_sync", err, err_len) ? 1 : 0;
}

int qw35_hip_runtime_buffer(void* runtime, uint32_t which, float** device_ptr, uint64_t* width, char* err,
                            uintptr_t err_len) {
    Runtime* r = static_cast<Runtime*>(runtime);
    if (!r || !device_ptr || !width) {
        rt_err(err, err_len, "runtime_buffer: invalid runtime or output pointers");
        return 0;
    }
    if (which >= QW35_HIP_RT_NBUF) {
        rt_err(err, err_len, "runtime_buffer: unknown buffer %u", which);
        return 0;
    }
    *device_ptr = r->buf[which];
    *width = r->width[which];
    return 1;
}

void* qw35_hip_runtime_stream(void* runtime) { return runtime ? static_cast<Runtime*>(runtime)->stream : nullptr; }

const void* qw35_hip_runtime_store(void* runtime) {
    return runtime ? static_cast<Runtime*>(runtime)->store : nullptr;
}

}  // extern "C"
