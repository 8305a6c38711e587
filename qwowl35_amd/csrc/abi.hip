// extern "C" entry points of include/qw35_hip.h: argument validation, the
// type-id -> kernel dispatch of encodeDecodeMatvecTensor
// (qw35-server/src/metal/bridge/Qw35MetalRuntime+FFN.m:184-256), the greedy
// head of encodeOutputHead (Qw35MetalRuntime+Output.m:11-65) and the
// 0 + err[err_len] error convention of Qw35FFI.m:15-22.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "../../include/qw35_hip.h"
#include "qw35_kernels.h"

namespace {

void set_err(char* err, uintptr_t err_len, const char* fmt, ...) {
    if (!err || err_len == 0) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, (size_t)err_len, fmt, ap);
    va_end(ap);
}

bool type_supported(uint32_t t) {
    return t == qw35::kTypeGF4 || t == qw35::kTypeGF2 || t == qw35::kTypeQ8_0 || t == qw35::kTypeQ4_K ||
           t == qw35::kTypeQ5_K ||
           t == qw35::kTypeQ6_K ||
           t == qw35::kTypeF16;
}

uint64_t row_bytes(uint32_t t, uint64_t k) {
    switch (t) {
        case qw35::kTypeGF4: return (k + 7) / 8 * 4;
        case qw35::kTypeGF2: return (k + 15) / 16 * 5;
        case qw35::kTypeQ8_0: return (k + 31) / 32 * 34;
        case qw35::kTypeQ4_K: return (k + 255) / 256 * 144;
        case qw35::kTypeQ5_K: return (k + 255) / 256 * 176;
        case qw35::kTypeQ6_K: return (k + 255) / 256 * 210;
        case qw35::kTypeF16: return k * 2;
        default: return 0;
    }
}

const char* type_name(uint32_t t) {
    switch (t) {
        case qw35::kTypeGF4: return "gf4";
        case qw35::kTypeGF2: return "gf2";
        case qw35::kTypeQ8_0: return "q8_0";
        case qw35::kTypeQ4_K: return "q4_k";
        case qw35::kTypeQ5_K: return "q5_k";
        case qw35::kTypeQ6_K: return "q6_k";
        case qw35::kTypeF16: return "f16";
        default: return "unsupported";
    }
}

// Longest row: the GEMVs cover any k in rounds of their plan's chunks; 65536
// keeps every in-kernel byte offset of a 64-row tile and of the prefill's
// staged token rows within 32 bits.
constexpr uint64_t kMaxK = 65536;
// Largest n_tokens * k of a prefill call (its fp16 token rows span < 2^31 bytes).
constexpr uint64_t kMaxPrefillElems = 1ull << 30;

bool check_weight(const qw35_hip_weight* w, const char* what, char* err, uintptr_t err_len) {
    if (!w) {
        set_err(err, err_len, "%s: null weight", what);
        return false;
    }
    if (!type_supported(w->type_id)) {
        set_err(err, err_len, "%s: unsupported tensor type %u", what, w->type_id);
        return false;
    }
    if (!w->data) {
        set_err(err, err_len, "%s: null weight data", what);
        return false;
    }
    if (((uintptr_t)w->data & 15u) != 0) {
        set_err(err, err_len, "%s: weight data must be 16-byte aligned", what);
        return false;
    }
    // q8_0 blocks are 32 columns (rows of k % 256 != 0 take the row-wise GEMV
    // only); every other codec's super-block or word group spans 256
    const uint64_t kstep = w->type_id == qw35::kTypeQ8_0 ? 32 : 256;
    if (w->k == 0 || w->k % kstep != 0 || w->k > kMaxK) {
        set_err(err, err_len, "%s: k=%llu must be a positive multiple of %llu and <= %llu", what,
                (unsigned long long)w->k, (unsigned long long)kstep, (unsigned long long)kMaxK);
        return false;
    }
    if (w->rows == 0 || w->rows > 0x7fffffffull) {
        set_err(err, err_len, "%s: rows=%llu out of range", what, (unsigned long long)w->rows);
        return false;
    }
    if (w->type_id == qw35::kTypeQ6_K && (w->k % 512 != 0 || row_bytes(w->type_id, w->k) * w->rows % 16 != 0)) {
        // 210-byte super-blocks, read as the 16-byte segments that cover them: rows
        // start at 4-byte boundaries for k % 512 == 0, and a matrix of a multiple of
        // 16 bytes ends where the last row's last segment does
        set_err(err, err_len, "%s: q6_k needs k %% 512 == 0 and rows * row bytes %% 16 == 0, got k=%llu rows=%llu",
                what, (unsigned long long)w->k, (unsigned long long)w->rows);
        return false;
    }
    const uint64_t want = row_bytes(w->type_id, w->k) * w->rows;
    if (w->bytes != want) {
        set_err(err, err_len, "%s: %s tensor %llux%llu must be %llu bytes, got %llu", what, type_name(w->type_id),
                (unsigned long long)w->rows, (unsigned long long)w->k, (unsigned long long)want,
                (unsigned long long)w->bytes);
        return false;
    }
    return true;
}

// The prefill matmul and the greedy head work in 256-column chunks.
bool check_chunked_k(const qw35_hip_weight* w, const char* what, char* err, uintptr_t err_len) {
    if (w->k % 256 == 0) return true;
    set_err(err, err_len, "%s: needs k %% 256 == 0, got k=%llu (a q8_0 weight of such k runs the decode GEMV only)",
            what, (unsigned long long)w->k);
    return false;
}

bool check_hip(hipError_t e, const char* what, char* err, uintptr_t err_len) {
    if (e == hipSuccess) return true;
    set_err(err, err_len, "%s: %s", what, hipGetErrorString(e));
    return false;
}

hipError_t dispatch_gemv(uint32_t type_id, const qw35::GemvArgs& a, hipStream_t s) {
    switch (type_id) {
        case qw35::kTypeGF4: return qw35::launch_gf4_gemv(a, s);
        case qw35::kTypeQ8_0: return qw35::launch_q8_0_gemv(a, s);
        case qw35::kTypeQ5_K: return qw35::launch_q5_k_gemv(a, s);
        case qw35::kTypeGF2: return qw35::launch_gf2_gemv(a, s);
        case qw35::kTypeQ6_K: return qw35::launch_q6_k_gemv(a, s);
        default: return qw35::launch_q4_k_gemv(a, s);
    }
}

// F16 tensors are prefill images: the GEMV kernels take the quantised bytes.
bool check_gemv_type(const qw35_hip_weight* w, const char* what, char* err, uintptr_t err_len) {
    if (w->type_id == qw35::kTypeF16) {
        set_err(err, err_len, "%s: f16 weights serve the prefill matmul only (the GEMVs take gf4/q8_0/q4_k/q6_k)",
                what);
        return false;
    }
    return true;
}

bool check_matvec(const qw35_hip_weight* w, const float* x, const float* awq, const float* dst, uint32_t n_batch,
                  const char* what, char* err, uintptr_t err_len) {
    if (!check_weight(w, what, err, err_len) || !check_gemv_type(w, what, err, err_len)) return false;
    if (!x || !dst) {
        set_err(err, err_len, "%s: null input or output", what);
        return false;
    }
    if (((uintptr_t)x & 15u) || (awq && ((uintptr_t)awq & 15u)) || ((uintptr_t)dst & 3u)) {
        set_err(err, err_len, "%s: x/awq must be 16-byte aligned and dst 4-byte aligned", what);
        return false;
    }
    if (n_batch < 1 || n_batch > QW35_HIP_MAX_BATCH) {
        set_err(err, err_len, "%s: n_batch=%u must be in 1..%u", what, n_batch, QW35_HIP_MAX_BATCH);
        return false;
    }
    return true;
}

bool check_swiglu(const qw35_hip_weight* gate, const qw35_hip_weight* up, const float* x, const float* awq,
                  const float* dst, uint32_t n_batch, const char* what, char* err, uintptr_t err_len) {
    if (!check_matvec(gate, x, awq, dst, n_batch, what, err, err_len)) return false;
    if (!check_weight(up, what, err, err_len)) return false;
    if (gate->type_id != up->type_id || gate->k != up->k || gate->rows != up->rows) {
        set_err(err, err_len, "%s: gate and up must share type and shape", what);
        return false;
    }
    if (gate->type_id == qw35::kTypeQ6_K) {
        set_err(err, err_len, "%s: q6_k has no fused gate/up form", what);
        return false;
    }
    return true;
}

qw35::GemvArgs gemv_args(const qw35_hip_weight* w, const qw35_hip_weight* up, const float* x, const float* awq,
                         float* dst, uint32_t n_batch, int residual) {
    qw35::GemvArgs a{};
    a.w = w->data;
    a.w_up = up ? up->data : nullptr;
    a.x = x;
    a.awq = awq;
    a.y = dst;
    a.rows = (int)w->rows;
    a.k = (int)w->k;
    a.n_batch = (int)n_batch;
    a.residual = residual ? 1 : 0;
    return a;
}

// Two plan ops can share one launch: both matvecs of the same k-quant type and
// k over the same activations, batch and AWQ, with the same residual flag,
// writing disjoint outputs that neither reads.
bool overlaps(const void* p, uint64_t pn, const void* q, uint64_t qn) {
    const uintptr_t a = (uintptr_t)p, b = (uintptr_t)q;
    return a < b + qn && b < a + pn;
}

bool mergeable(const qw35_hip_plan_op& a, const qw35_hip_plan_op& b) {
    if (a.kind != QW35_HIP_OP_MATVEC || b.kind != QW35_HIP_OP_MATVEC) return false;
    if (b.w->type_id != a.w->type_id || b.w->k != a.w->k || b.x != a.x || b.awq != a.awq ||
        b.n_batch != a.n_batch || (b.residual != 0) != (a.residual != 0))
        return false;
    const uint64_t xa = (uint64_t)a.n_batch * a.w->k * 4;
    const uint64_t da = (uint64_t)a.n_batch * a.w->rows * 4, db = (uint64_t)b.n_batch * b.w->rows * 4;
    return !overlaps(a.dst, da, b.dst, db) && !overlaps(a.x, xa, a.dst, da) && !overlaps(a.x, xa, b.dst, db);
}

// What a prefill launch staged into its workspace: the activations, AWQ,
// token count, k and column order (GF4 words take their own order).
struct StageKey {
    const float* x = nullptr;
    const float* awq = nullptr;
    const void* ws = nullptr;
    uint32_t n = 0, k = 0;
    bool gf4_order = false;
    bool operator==(const StageKey& o) const {
        return x == o.x && awq == o.awq && ws == o.ws && n == o.n && k == o.k && gf4_order == o.gf4_order;
    }
};

// Weight form of the prefill kernel: 0 GF4 words, 1 F16, 2 q8_0 blocks, 3 Q4_K super-blocks; -1 none.
int prefill_wkind(uint32_t type_id) {
    return type_id == qw35::kTypeGF4    ? 0
           : type_id == qw35::kTypeF16  ? 1
           : type_id == qw35::kTypeQ8_0 ? 2
           : type_id == qw35::kTypeQ4_K ? 3
                                        : -1;
}

// A MATMUL / MATMUL_SWIGLU plan op: the rules of qw35_hip_matmul_prefill(_epilogue)
// with fp32 activations and output and the op's workspace.
bool check_matmul_op(const qw35_hip_plan_op& o, const char* what, char* err, uintptr_t err_len) {
    const bool sw = o.kind == QW35_HIP_OP_MATMUL_SWIGLU;
    if (!check_weight(o.w, what, err, err_len) || !check_chunked_k(o.w, what, err, err_len)) return false;
    if (prefill_wkind(o.w->type_id) < 0) {
        set_err(err, err_len, "%s: the prefill matmul takes GF4, q8_0, Q4_K or F16 weights, got type %u", what,
                o.w->type_id);
        return false;
    }
    if (sw) {
        if (o.residual) {
            set_err(err, err_len, "%s: a MATMUL_SWIGLU op has no residual form", what);
            return false;
        }
        if (!check_weight(o.w_up, what, err, err_len)) return false;
        if (o.w_up->type_id != o.w->type_id || o.w_up->k != o.w->k || o.w_up->rows != o.w->rows) {
            set_err(err, err_len, "%s: gate and up must share type and shape", what);
            return false;
        }
    } else if (o.w_up) {
        set_err(err, err_len, "%s: a MATMUL op takes no w_up", what);
        return false;
    }
    if (!o.x || !o.dst || ((uintptr_t)o.x & 15u) || (o.awq && ((uintptr_t)o.awq & 15u)) || ((uintptr_t)o.dst & 3u)) {
        set_err(err, err_len, "%s: x/awq must be non-null 16-byte aligned and dst non-null 4-byte aligned", what);
        return false;
    }
    if (o.n_batch < 1 || o.n_batch > 65536 || (uint64_t)o.n_batch * o.w->k > kMaxPrefillElems / 2 ||
        o.w->rows > (1ull << 24)) {
        set_err(err, err_len, "%s: n_batch=%u tokens must be in 1..65536 with n_batch * k <= %llu", what, o.n_batch,
                (unsigned long long)(kMaxPrefillElems / 2));
        return false;
    }
    const uint64_t need = qw35::prefill_min_workspace_bytes((int)o.n_batch, (int)o.w->rows, (int)o.w->k, true);
    if (!o.workspace || ((uintptr_t)o.workspace & 255u) || o.workspace_bytes < need) {
        set_err(err, err_len, "%s: a MATMUL op needs a 256-byte aligned workspace of >= %llu bytes", what,
                (unsigned long long)need);
        return false;
    }
    return true;
}

// Consecutive MATMUL ops over the same activations (a mixer's input
// projections) share one prefill launch: same weight form and k, same x, AWQ,
// token count, workspace and epilogue, row counts that are multiples of 4, and
// no op's output overlapping another's or the shared inputs.
bool prefill_mergeable(const qw35_hip_plan_op& a, const qw35_hip_plan_op& b) {
    if (a.kind != QW35_HIP_OP_MATMUL || b.kind != QW35_HIP_OP_MATMUL) return false;
    if (prefill_wkind(b.w->type_id) != prefill_wkind(a.w->type_id) || b.w->k != a.w->k || b.x != a.x ||
        b.awq != a.awq || b.n_batch != a.n_batch || b.workspace != a.workspace ||
        b.workspace_bytes != a.workspace_bytes || (b.residual != 0) != (a.residual != 0) || a.w->rows % 4 != 0 ||
        b.w->rows % 4 != 0)
        return false;
    const uint64_t xa = (uint64_t)a.n_batch * a.w->k * 4, wa = a.awq ? a.w->k * 4 : 0;
    const uint64_t da = (uint64_t)a.n_batch * a.w->rows * 4, db = (uint64_t)b.n_batch * b.w->rows * 4;
    return !overlaps(a.dst, da, b.dst, db) && !overlaps(a.x, xa, a.dst, da) && !overlaps(a.x, xa, b.dst, db) &&
           !(a.awq && (overlaps(a.awq, wa, a.dst, da) || overlaps(a.awq, wa, b.dst, db)));
}

// Greedy head workspace: per batch row, one (token, logit) partial per
// workgroup of the GEMV launch; tokens first, logits at a 256-byte boundary.
uint64_t argmax_ws_part(const qw35_hip_weight* w, uint32_t n_batch) {
    const uint64_t n = (uint64_t)qw35::argmax_groups(w->type_id, (int)w->rows, (int)w->k, (int)n_batch) * n_batch;
    return (n * 4 + 255) / 256 * 256;
}

// A recorded decode-step plan: the launches (their weight pointers, shapes and
// buffers baked into the kernel arguments) held as an instantiated hipGraph.
struct Plan {
    uint32_t n_ops = 0;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    void* ws = nullptr;  // K-split workspace shared by the plan's launches (they run in order)
};

void plan_free(Plan* p) {
    if (!p) return;
    if (p->exec) (void)hipGraphExecDestroy(p->exec);
    if (p->graph) (void)hipGraphDestroy(p->graph);
    if (p->ws) (void)hipFree(p->ws);
    delete p;
}

}  // namespace

extern "C" {

int qw35_hip_has_device(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n > 0 ? 1 : 0;
}

int qw35_hip_weight_view(const qw35_hip_tensor_desc* desc, const void* device_base, qw35_hip_weight* out, char* err,
                         uintptr_t err_len) {
    if (!desc || !out) {
        set_err(err, err_len, "weight_view: null descriptor or output");
        return 0;
    }
    if (!device_base) {
        set_err(err, err_len, "weight_view: null device base");
        return 0;
    }
    if (desc->n_dims < 2) {
        set_err(err, err_len, "weight_view: tensor is not a matrix (n_dims=%u)", desc->n_dims);
        return 0;
    }
    for (uint32_t i = 2; i < desc->n_dims && i < 4; ++i) {
        if (desc->dims[i] != 1) {
            set_err(err, err_len, "weight_view: dims[%u]=%llu, only 2-D weights are supported", i,
                    (unsigned long long)desc->dims[i]);
            return 0;
        }
    }
    if (desc->elements != desc->dims[0] * desc->dims[1]) {
        set_err(err, err_len, "weight_view: elements=%llu != dims[0]*dims[1]", (unsigned long long)desc->elements);
        return 0;
    }
    qw35_hip_weight w;
    w.data = static_cast<const uint8_t*>(device_base) + desc->abs_offset;
    w.k = desc->dims[0];
    w.rows = desc->dims[1];
    w.bytes = desc->bytes;
    w.type_id = desc->type_id;
    w.reserved = 0;
    if (!check_weight(&w, "weight_view", err, err_len)) return 0;
    *out = w;
    return 1;
}

int qw35_hip_decode_matvec(const qw35_hip_weight* w, const float* x, const float* awq, float* dst,
                           uint32_t n_batch, int residual, void* stream, char* err, uintptr_t err_len) {
    if (!check_matvec(w, x, awq, dst, n_batch, "decode_matvec", err, err_len)) return 0;
    const qw35::GemvArgs a = gemv_args(w, nullptr, x, awq, dst, n_batch, residual);
    return check_hip(dispatch_gemv(w->type_id, a, static_cast<hipStream_t>(stream)), "decode_matvec", err, err_len)
               ? 1
               : 0;
}

int qw35_hip_ffn_gate_up_swiglu(const qw35_hip_weight* gate, const qw35_hip_weight* up, const float* x,
                                const float* awq, float* dst, uint32_t n_batch, void* stream, char* err,
                                uintptr_t err_len) {
    if (!check_swiglu(gate, up, x, awq, dst, n_batch, "ffn_gate_up_swiglu", err, err_len)) return 0;
    const qw35::GemvArgs a = gemv_args(gate, up, x, awq, dst, n_batch, 0);
    return check_hip(dispatch_gemv(gate->type_id, a, static_cast<hipStream_t>(stream)), "ffn_gate_up_swiglu", err,
                     err_len)
               ? 1
               : 0;
}

int qw35_hip_gemv_kernel(const qw35_hip_weight* w, const qw35_hip_weight* w_up, uint32_t n_batch, int has_awq,
                         int with_workspace, char* name, uintptr_t name_len, uint32_t* grid, uint32_t* block,
                         uint32_t* lds_bytes, uint64_t* workspace_bytes, char* err, uintptr_t err_len) {
    // Stand-in addresses for the validation: nothing is launched or read.
    const float* fake = reinterpret_cast<const float*>(uintptr_t{256});
    const float* awq = has_awq ? fake : nullptr;
    float* dst = const_cast<float*>(fake);
    const bool ok = w_up ? check_swiglu(w, w_up, fake, awq, dst, n_batch, "gemv_kernel", err, err_len)
                         : check_matvec(w, fake, awq, dst, n_batch, "gemv_kernel", err, err_len);
    if (!ok) return 0;
    qw35::LaunchInfo info{};
    info.splits = 1;
    qw35::GemvArgs a = gemv_args(w, w_up, fake, awq, dst, n_batch, 0);
    a.info = &info;
    if (with_workspace) {  // a workspace large enough for any plan
        a.ks_ws = const_cast<float*>(fake);
        a.ks_ws_bytes = UINT64_MAX;
    }
    if (!check_hip(dispatch_gemv(w->type_id, a, nullptr), "gemv_kernel", err, err_len)) return 0;
    if (name && name_len) snprintf(name, (size_t)name_len, "%s", info.name);
    if (grid) *grid = info.grid;
    if (block) *block = info.block;
    if (lds_bytes) *lds_bytes = info.lds;
    if (workspace_bytes) *workspace_bytes = info.ws_bytes;
    return 1;
}

uint64_t qw35_hip_decode_matvec_workspace_size(const qw35_hip_weight* w, uint32_t n_batch) {
    char msg[8];
    uint64_t bytes = 0;
    if (!qw35_hip_gemv_kernel(w, nullptr, n_batch, 0, 1, nullptr, 0, nullptr, nullptr, nullptr, &bytes, msg,
                              sizeof msg))
        return 0;
    return bytes;
}

int qw35_hip_decode_matvec_ws(const qw35_hip_weight* w, const float* x, const float* awq, float* dst,
                              uint32_t n_batch, int residual, void* workspace, uint64_t workspace_bytes, void* stream,
                              char* err, uintptr_t err_len) {
    if (!check_matvec(w, x, awq, dst, n_batch, "decode_matvec_ws", err, err_len)) return 0;
    if (workspace && ((uintptr_t)workspace & 255u)) {
        set_err(err, err_len, "decode_matvec_ws: workspace must be 256-byte aligned");
        return 0;
    }
    qw35::GemvArgs a = gemv_args(w, nullptr, x, awq, dst, n_batch, residual);
    a.ks_ws = workspace;
    a.ks_ws_bytes = workspace ? workspace_bytes : 0;
    return check_hip(dispatch_gemv(w->type_id, a, static_cast<hipStream_t>(stream)), "decode_matvec_ws", err,
                     err_len)
               ? 1
               : 0;
}

void* qw35_hip_plan_create(const qw35_hip_plan_op* ops, uint32_t n_ops, char* err, uintptr_t err_len) {
    if (!ops || n_ops == 0) {
        set_err(err, err_len, "plan_create: no ops");
        return nullptr;
    }
    char what[64];
    for (uint32_t i = 0; i < n_ops; ++i) {
        const qw35_hip_plan_op& o = ops[i];
        snprintf(what, sizeof what, "plan_create: op %u", i);
        if (o.kind == QW35_HIP_OP_MATVEC) {
            if (o.w_up) {
                set_err(err, err_len, "%s: a MATVEC op takes no w_up", what);
                return nullptr;
            }
            if (!check_matvec(o.w, o.x, o.awq, o.dst, o.n_batch, what, err, err_len)) return nullptr;
        } else if (o.kind == QW35_HIP_OP_SWIGLU) {
            if (o.residual) {
                set_err(err, err_len, "%s: a SWIGLU op has no residual form", what);
                return nullptr;
            }
            if (!check_swiglu(o.w, o.w_up, o.x, o.awq, o.dst, o.n_batch, what, err, err_len)) return nullptr;
        } else if (o.kind == QW35_HIP_OP_ARGMAX) {
            if (o.w_up || o.residual) {
                set_err(err, err_len, "%s: an ARGMAX op takes no w_up or residual", what);
                return nullptr;
            }
            if (!check_matvec(o.w, o.x, o.awq, o.dst, o.n_batch, what, err, err_len) ||
                !check_chunked_k(o.w, what, err, err_len))
                return nullptr;
            if (!o.token || ((uintptr_t)o.token & 3u)) {
                set_err(err, err_len, "%s: an ARGMAX op needs a 4-byte aligned token output", what);
                return nullptr;
            }
            const uint64_t part = argmax_ws_part(o.w, o.n_batch);
            if (!o.workspace || ((uintptr_t)o.workspace & 255u) || o.workspace_bytes < 2 * part) {
                set_err(err, err_len, "%s: an ARGMAX op needs a 256-byte aligned workspace of >= %llu bytes", what,
                        (unsigned long long)(2 * part));
                return nullptr;
            }
        } else if (o.kind == QW35_HIP_OP_MATMUL || o.kind == QW35_HIP_OP_MATMUL_SWIGLU) {
            if (!check_matmul_op(o, what, err, err_len)) return nullptr;
        } else {
            set_err(err, err_len, "%s: unknown kind %u", what, o.kind);
            return nullptr;
        }
    }
    Plan* plan = new Plan();
    plan->n_ops = n_ops;
    // Size the K-split workspace for the launches (described, not launched),
    // then allocate and zero it once, outside the capture: the launches run in
    // order and each returns its counters to zero.
    uint64_t ws_bytes = 0;
    hipError_t launch = hipSuccess;
    for (int pass = 0; pass < 2 && launch == hipSuccess; ++pass) {
        hipStream_t s = nullptr;
        hipError_t e = hipSuccess;
        if (pass == 1) {
            if (ws_bytes) {
                e = hipMalloc(&plan->ws, ws_bytes);
                if (e == hipSuccess) e = hipMemset(plan->ws, 0, ws_bytes);
                // the counters must be zero before the first replay, on whatever stream it runs
                if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
            }
            if (e == hipSuccess) e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
            if (e == hipSuccess) e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
            if (e != hipSuccess) {
                if (s) (void)hipStreamDestroy(s);
                check_hip(e, "plan_create: workspace / stream", err, err_len);
                plan_free(plan);
                return nullptr;
            }
        }
        qw35::LaunchInfo info{};
        StageKey stage_key{};
        bool stage_valid = false;
        for (uint32_t i = 0; i < n_ops && launch == hipSuccess;) {
            const qw35_hip_plan_op& o = ops[i];
            if (o.kind == QW35_HIP_OP_MATMUL || o.kind == QW35_HIP_OP_MATMUL_SWIGLU) {
                const bool sw = o.kind == QW35_HIP_OP_MATMUL_SWIGLU;
                // ops [i, j) run as one launch (segments) when mergeable
                uint32_t j = i + 1;
                while (!sw && j < n_ops && j - i < (uint32_t)qw35::kMaxSegments) {
                    bool ok = true;
                    for (uint32_t q = i; q < j && ok; ++q) ok = prefill_mergeable(ops[q], ops[j]);
                    if (!ok) break;
                    ++j;
                }
                if (pass == 1) {
                    qw35::PrefillSegs segs;
                    uint64_t rows = o.w->rows;
                    if (j - i > 1) {
                        segs.n = (int)(j - i);
                        rows = 0;
                        for (uint32_t q = i; q < j; ++q) {
                            segs.w[q - i] = ops[q].w->data;
                            segs.c[q - i] = ops[q].dst;
                            segs.rows[q - i] = (int)ops[q].w->rows;
                            rows += ops[q].w->rows;
                        }
                    }
                    auto mm = [&](const qw35_hip_weight* w, uint32_t epi, const qw35_hip_weight* w_up) {
                        // The staging pass is skipped when the previous prefill launch
                        // of the plan staged the same activations the same way into
                        // the same workspace, and nothing written since overlaps them.
                        const int wkind = prefill_wkind(w->type_id);
                        const StageKey key{o.x, o.awq, o.workspace, o.n_batch, (uint32_t)w->k, wkind == 0};
                        const bool staged = stage_valid && key == stage_key;
                        const bool multi = segs.n > 1 && w == o.w;
                        const hipError_t e = qw35::launch_prefill(
                            wkind, w->data, multi ? (int)rows : (int)w->rows, (int)w->k, o.x, 1, o.awq, o.dst,
                            (int)o.n_batch, 1, o.workspace, o.workspace_bytes, s, (int)epi, nullptr, staged,
                            multi ? &segs : nullptr, w_up ? w_up->data : nullptr);
                        stage_key = key;
                        // this launch's outputs may be the next one's input
                        const uint64_t xb = (uint64_t)o.n_batch * w->k * 4;
                        stage_valid = true;
                        for (uint32_t q = i; q < (multi ? j : i + 1); ++q) {
                            const uint64_t db = (uint64_t)o.n_batch * ops[q].w->rows * 4;
                            const void* d = multi ? ops[q].dst : o.dst;
                            if (overlaps(d, db, o.x, xb) || (o.awq && overlaps(d, db, o.awq, w->k * 4)))
                                stage_valid = false;
                        }
                        return e;
                    };
                    // gate/up: one fused launch where plan_swiglu finds a fused tile for it
                    const bool fused = sw && qw35::prefill_swiglu_fusable(prefill_wkind(o.w->type_id), (int)o.n_batch,
                                                                          (int)o.w->rows, (int)o.w->k, 1,
                                                                          o.workspace_bytes);
                    launch = mm(o.w, sw          ? QW35_HIP_EPILOGUE_STORE
                                     : o.residual ? QW35_HIP_EPILOGUE_ADD
                                                  : QW35_HIP_EPILOGUE_STORE,
                                fused ? o.w_up : nullptr);
                    if (launch == hipSuccess && sw && !fused) launch = mm(o.w_up, QW35_HIP_EPILOGUE_SWIGLU, nullptr);
                }
                i = j;
                continue;
            }
            stage_valid = false;  // GEMV outputs are not tracked against the staged activations
            if (o.kind == QW35_HIP_OP_ARGMAX) {
                qw35::GemvArgs a = gemv_args(o.w, nullptr, o.x, o.awq, nullptr, o.n_batch, 0);
                a.am_token = static_cast<uint32_t*>(o.workspace);
                a.am_logit = reinterpret_cast<float*>(static_cast<uint8_t*>(o.workspace) +
                                                      argmax_ws_part(o.w, o.n_batch));
                if (pass == 1) launch = qw35::launch_argmax_gemv(o.w->type_id, a, o.token, o.dst, s);
                ++i;
                continue;
            }
            const bool sw = o.kind == QW35_HIP_OP_SWIGLU;
            qw35::GemvArgs a = gemv_args(o.w, sw ? o.w_up : nullptr, o.x, o.awq, o.dst, o.n_batch,
                                         sw ? 0 : o.residual);
            // Consecutive k-quant matvecs over the same activations share one launch.
            uint32_t j = i + 1;
            if (!sw && o.w->type_id != qw35::kTypeGF4) {
                while (j < n_ops && j - i < (uint32_t)qw35::kMaxSegments) {
                    bool ok = true;
                    for (uint32_t q = i; q < j && ok; ++q) ok = mergeable(ops[q], ops[j]);
                    if (!ok) break;
                    ++j;
                }
            }
            if (j - i > 1) {
                a.n_seg = (int)(j - i);
                for (uint32_t q = i; q < j; ++q) {
                    a.seg_w[q - i] = ops[q].w->data;
                    a.seg_y[q - i] = ops[q].dst;
                    a.seg_rows[q - i] = (int)ops[q].w->rows;
                }
            }
            if (pass == 0) {  // describe with an unbounded workspace: the bytes this launch would use
                a.info = &info;
                a.ks_ws = reinterpret_cast<void*>(uintptr_t{256});
                a.ks_ws_bytes = UINT64_MAX;
                info.ws_bytes = 0;
                launch = dispatch_gemv(o.w->type_id, a, nullptr);
                if (info.ws_bytes > ws_bytes) ws_bytes = info.ws_bytes;
            } else {
                a.ks_ws = plan->ws;
                a.ks_ws_bytes = ws_bytes;
                launch = dispatch_gemv(o.w->type_id, a, s);
            }
            i = j;
        }
        if (pass == 1) {
            e = hipStreamEndCapture(s, &plan->graph);
            if (e == hipSuccess) e = launch;
            if (e == hipSuccess) e = hipGraphInstantiate(&plan->exec, plan->graph, nullptr, nullptr, 0);
            (void)hipStreamDestroy(s);
            if (!check_hip(e, "plan_create: record", err, err_len)) {
                plan_free(plan);
                return nullptr;
            }
        }
    }
    if (!check_hip(launch, "plan_create: describe", err, err_len)) {
        plan_free(plan);
        return nullptr;
    }
    return plan;
}

int qw35_hip_plan_launch(void* plan, void* stream, char* err, uintptr_t err_len) {
    if (!plan) {
        set_err(err, err_len, "plan_launch: null plan");
        return 0;
    }
    return check_hip(hipGraphLaunch(static_cast<Plan*>(plan)->exec, static_cast<hipStream_t>(stream)),
                     "plan_launch", err, err_len)
               ? 1
               : 0;
}

uint32_t qw35_hip_plan_size(const void* plan) { return plan ? static_cast<const Plan*>(plan)->n_ops : 0u; }

void qw35_hip_plan_destroy(void* plan) { plan_free(static_cast<Plan*>(plan)); }

int qw35_hip_dequantize(const qw35_hip_weight* w, const uint32_t* row_ids, uint32_t n_rows, float* dst, void* stream,
                        char* err, uintptr_t err_len) {
    if (!check_weight(w, "dequantize", err, err_len)) return 0;
    if (!dst) {
        set_err(err, err_len, "dequantize: null output");
        return 0;
    }
    if ((uintptr_t)dst & 15u) {
        set_err(err, err_len, "dequantize: dst must be 16-byte aligned");
        return 0;
    }
    const int out_rows = row_ids ? (int)n_rows : (int)w->rows;
    if (row_ids && n_rows > 0x7fffffffu) {
        set_err(err, err_len, "dequantize: n_rows out of range");
        return 0;
    }
    return check_hip(qw35::launch_dequant(w->type_id, w->data, (int)w->rows, (int)w->k, row_ids, out_rows, dst,
                                          false, static_cast<hipStream_t>(stream)),
                     "dequantize", err, err_len)
               ? 1
               : 0;
}

int qw35_hip_dequantize_f16(const qw35_hip_weight* w, void* dst, void* stream, char* err, uintptr_t err_len) {
    if (!check_weight(w, "dequantize_f16", err, err_len)) return 0;
    if (!dst || ((uintptr_t)dst & 15u)) {
        set_err(err, err_len, "dequantize_f16: dst must be non-null and 16-byte aligned");
        return 0;
    }
    return check_hip(qw35::launch_dequant(w->type_id, w->data, (int)w->rows, (int)w->k, nullptr, (int)w->rows, dst,
                                          true, static_cast<hipStream_t>(stream)),
                     "dequantize_f16", err, err_len)
               ? 1
               : 0;
}

uint64_t qw35_hip_matmul_prefill_workspace_size(const qw35_hip_weight* w, uint32_t n_tokens) {
    char msg[8];
    if (!check_weight(w, "matmul_prefill", msg, sizeof msg) || !check_chunked_k(w, "", msg, sizeof msg) ||
        n_tokens < 1 || n_tokens > 65536 || (uint64_t)n_tokens * w->k > kMaxPrefillElems)
        return 0;
    const int wkind = prefill_wkind(w->type_id);
    if (wkind < 0) return 0;
    // fp32 activations (two staged rows per token) are accepted up to half the elements
    return (uint64_t)qw35::prefill_workspace_bytes((int)n_tokens, (int)w->rows, (int)w->k, wkind,
                                                   (uint64_t)n_tokens * w->k <= kMaxPrefillElems / 2);
}

int qw35_hip_matmul_prefill(const qw35_hip_weight* w, const void* a, uint32_t a_dtype, const float* awq, void* c,
                            uint32_t c_dtype, uint32_t n_tokens, void* workspace, uint64_t workspace_bytes,
                            void* stream, char* err, uintptr_t err_len) {
    return qw35_hip_matmul_prefill_epilogue(w, a, a_dtype, awq, c, c_dtype, QW35_HIP_EPILOGUE_STORE, n_tokens,
                                            workspace, workspace_bytes, stream, err, err_len);
}

// The checks of a prefill call, then its launch, or (info set) its description.
static int prefill_call(const qw35_hip_weight* w, const void* a, uint32_t a_dtype, const float* awq, void* c,
                        uint32_t c_dtype, uint32_t epilogue, uint32_t n_tokens, void* workspace,
                        uint64_t workspace_bytes, void* stream, qw35::LaunchInfo* info, char* err, uintptr_t err_len) {
    if (!check_weight(w, "matmul_prefill", err, err_len) || !check_chunked_k(w, "matmul_prefill", err, err_len))
        return 0;
    if (epilogue > QW35_HIP_EPILOGUE_SWIGLU) {
        set_err(err, err_len, "matmul_prefill: unknown epilogue %u", epilogue);
        return 0;
    }
    if (epilogue != QW35_HIP_EPILOGUE_STORE && (c_dtype != QW35_HIP_DTYPE_F32 || !workspace)) {
        set_err(err, err_len, "matmul_prefill: the add and SwiGLU epilogues take fp32 c and a workspace");
        return 0;
    }
    if (prefill_wkind(w->type_id) < 0) {
        set_err(err, err_len,
                "matmul_prefill: GF4 (type 100), q8_0 (type 8), Q4_K (type 12) or F16 (type 1) weights, got %s; make the fp16 "
                "prefill image of another k-quant weight with qw35_hip_dequantize_f16",
                type_name(w->type_id));
        return 0;
    }
    if (a_dtype > QW35_HIP_DTYPE_BF16 || c_dtype > QW35_HIP_DTYPE_BF16) {
        set_err(err, err_len, "matmul_prefill: a_dtype/c_dtype must be QW35_HIP_DTYPE_F32 or QW35_HIP_DTYPE_BF16");
        return 0;
    }
    if (n_tokens < 1 || n_tokens > 65536) {
        set_err(err, err_len, "matmul_prefill: n_tokens=%u must be in 1..65536", n_tokens);
        return 0;
    }
    // staged token offsets are 32-bit byte offsets; fp32 input stages two rows per token
    const uint64_t max_elems = a_dtype == QW35_HIP_DTYPE_F32 ? kMaxPrefillElems / 2 : kMaxPrefillElems;
    if ((uint64_t)n_tokens * w->k > max_elems) {
        set_err(err, err_len, "matmul_prefill: n_tokens * k = %llu must be <= %llu for %s activations",
                (unsigned long long)n_tokens * w->k, (unsigned long long)max_elems,
                a_dtype == QW35_HIP_DTYPE_F32 ? "fp32" : "bf16");
        return 0;
    }
    if (w->rows > (1ull << 24)) {  // keeps every launch grid within 2^31 blocks
        set_err(err, err_len, "matmul_prefill: rows=%llu must be <= 16777216", (unsigned long long)w->rows);
        return 0;
    }
    if (!a || !c) {
        set_err(err, err_len, "matmul_prefill: null input or output");
        return 0;
    }
    if (((uintptr_t)a & 15u) || (awq && ((uintptr_t)awq & 15u)) || ((uintptr_t)c & 3u)) {
        set_err(err, err_len, "matmul_prefill: a/awq must be 16-byte aligned and c 4-byte aligned");
        return 0;
    }
    const int wkind = prefill_wkind(w->type_id);
    const bool a_f32 = a_dtype == QW35_HIP_DTYPE_F32;
    if (!workspace && wkind == 0 && (a_f32 || awq)) {
        set_err(err, err_len,
                "matmul_prefill: fp32 activations and AWQ need a workspace (the staged path); the path without one "
                "contracts bf16 operands and takes bf16 activations without AWQ only");
        return 0;
    }
    if (workspace || wkind != 0) {
        const uint64_t need = qw35::prefill_min_workspace_bytes((int)n_tokens, (int)w->rows, (int)w->k, a_f32);
        if (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 255u)) {
            set_err(err, err_len,
                    "matmul_prefill: %s a 256-byte aligned workspace of >= %llu bytes for %u %s tokens, got %llu",
                    wkind == 0   ? "the staged path needs"
                    : wkind == 1 ? "f16 weights need"
                    : wkind == 2 ? "q8_0 weights need"
                                 : "q4_k weights need",
                    (unsigned long long)need, n_tokens, a_f32 ? "fp32" : "bf16",
                    (unsigned long long)(workspace ? workspace_bytes : 0));
            return 0;
        }
    }
    return check_hip(qw35::launch_prefill(wkind, w->data, (int)w->rows, (int)w->k, a, a_f32, awq, c, (int)n_tokens,
                                          c_dtype == QW35_HIP_DTYPE_F32, workspace, workspace ? workspace_bytes : 0,
                                          static_cast<hipStream_t>(stream), (int)epilogue, info),
                     "matmul_prefill", err, err_len)
               ? 1
               : 0;
}

int qw35_hip_matmul_prefill_epilogue(const qw35_hip_weight* w, const void* a, uint32_t a_dtype, const float* awq,
                                     void* c, uint32_t c_dtype, uint32_t epilogue, uint32_t n_tokens, void* workspace,
                                     uint64_t workspace_bytes, void* stream, char* err, uintptr_t err_len) {
    return prefill_call(w, a, a_dtype, awq, c, c_dtype, epilogue, n_tokens, workspace, workspace_bytes, stream,
                        nullptr, err, err_len);
}

int qw35_hip_prefill_kernel(const qw35_hip_weight* w, uint32_t n_tokens, uint32_t a_dtype, int has_awq,
                            uint32_t c_dtype, int with_workspace, char* name, uintptr_t name_len, uint32_t* grid,
                            uint32_t* block, uint32_t* lds_bytes, uint32_t* splits, char* err, uintptr_t err_len) {
    // Stand-in addresses for the validation: nothing is launched or read.
    void* fake = reinterpret_cast<void*>(uintptr_t{256});
    qw35::LaunchInfo info{};
    info.splits = 1;
    if (!prefill_call(w, fake, a_dtype, has_awq ? static_cast<const float*>(fake) : nullptr, fake, c_dtype,
                      QW35_HIP_EPILOGUE_STORE, n_tokens, with_workspace ? fake : nullptr,
                      with_workspace ? UINT64_MAX : 0, nullptr, &info, err, err_len))
        return 0;
    if (name && name_len) snprintf(name, (size_t)name_len, "%s", info.name);
    if (grid) *grid = info.grid;
    if (block) *block = info.block;
    if (lds_bytes) *lds_bytes = info.lds;
    if (splits) *splits = info.splits;
    return 1;
}

int qw35_hip_quantize(uint32_t type_id, const float* src, uint64_t rows, uint64_t k, const float* col_scale,
                      void* dst, void* stream, char* err, uintptr_t err_len) {
    if (!type_supported(type_id)) {
        set_err(err, err_len, "quantize: unsupported tensor type %u", type_id);
        return 0;
    }
    const uint64_t block =
        (type_id == qw35::kTypeGF4 || type_id == qw35::kTypeF16) ? 8 : type_id == qw35::kTypeQ8_0 ? 32 : 256;
    if (k == 0 || k % block != 0 || k > 0x7fffffffull) {
        set_err(err, err_len, "quantize: k=%llu must be a positive multiple of %llu for %s",
                (unsigned long long)k, (unsigned long long)block, type_name(type_id));
        return 0;
    }
    if (rows == 0 || rows > 0x7fffffffull) {
        set_err(err, err_len, "quantize: rows=%llu out of range", (unsigned long long)rows);
        return 0;
    }
    if (!src || !dst) {
        set_err(err, err_len, "quantize: null input or output");
        return 0;
    }
    if (((uintptr_t)src & 15u) || ((uintptr_t)dst & 15u) || (col_scale && ((uintptr_t)col_scale & 15u))) {
        set_err(err, err_len, "quantize: src, dst and col_scale must be 16-byte aligned");
        return 0;
    }
    return check_hip(qw35::launch_quantize(type_id, src, (int)rows, (int)k, col_scale, dst,
                                           static_cast<hipStream_t>(stream)),
                     "quantize", err, err_len)
               ? 1
               : 0;
}


uint64_t qw35_hip_output_argmax_workspace_size(const qw35_hip_weight* w, uint32_t n_batch) {
    char msg[8];
    if (!check_weight(w, "output_argmax", msg, sizeof msg) || !check_chunked_k(w, "", msg, sizeof msg) ||
        w->type_id == qw35::kTypeF16 || n_batch < 1 || n_batch > QW35_HIP_MAX_BATCH)
        return 0;
    return 2 * argmax_ws_part(w, n_batch);
}

int qw35_hip_output_argmax(const qw35_hip_weight* w, const float* x, const float* awq, uint32_t n_batch,
                           uint32_t* token, float* logit, void* workspace, uint64_t workspace_bytes, void* stream,
                           char* err, uintptr_t err_len) {
    if (!check_weight(w, "output_argmax", err, err_len) || !check_gemv_type(w, "output_argmax", err, err_len) ||
        !check_chunked_k(w, "output_argmax", err, err_len))
        return 0;
    if (!x || !token || !logit || !workspace) {
        set_err(err, err_len, "output_argmax: null input, output or workspace");
        return 0;
    }
    if (((uintptr_t)x & 15u) || (awq && ((uintptr_t)awq & 15u)) || ((uintptr_t)token & 3u) || ((uintptr_t)logit & 3u)) {
        set_err(err, err_len, "output_argmax: x/awq must be 16-byte aligned, token/logit 4-byte aligned");
        return 0;
    }
    if (n_batch < 1 || n_batch > QW35_HIP_MAX_BATCH) {
        set_err(err, err_len, "output_argmax: n_batch=%u must be in 1..%u", n_batch, QW35_HIP_MAX_BATCH);
        return 0;
    }
    const uint64_t part = argmax_ws_part(w, n_batch);
    if (workspace_bytes < 2 * part || ((uintptr_t)workspace & 255u)) {
        set_err(err, err_len, "output_argmax: workspace must be 256-byte aligned and >= %llu bytes, got %llu",
                (unsigned long long)(2 * part), (unsigned long long)workspace_bytes);
        return 0;
    }
    qw35::GemvArgs a = gemv_args(w, nullptr, x, awq, nullptr, n_batch, 0);
    a.am_token = static_cast<uint32_t*>(workspace);
    a.am_logit = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + part);
    return check_hip(qw35::launch_argmax_gemv(w->type_id, a, token, logit, static_cast<hipStream_t>(stream)),
                     "output_argmax", err, err_len)
               ? 1
               : 0;
}

}  // extern "C"

// Scratch of qw35_hip_output_argmax_noalloc: the greedy head's per-workgroup
// (row, logit) partials, in a device array the library owns instead of a
// caller workspace.  Each GPU holds its own copy for the life of the process;
// host code addresses it only through the pointer hipGetSymbolAddress
// returns for the current device (the array's name is a host-side stand-in).
static __device__ __align__(256) uint8_t scratch[QW35_HIP_ARGMAX_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's copy of `scratch`, looked up once per device.
void* scratch_of_current_device(char* err, uintptr_t err_len) {
    int dev = -1;
    if (!check_hip(hipGetDevice(&dev), "output_argmax_noalloc: device", err, err_len)) return nullptr;
    if (dev < 0 || dev >= kMaxDevices) {
        set_err(err, err_len, "output_argmax_noalloc: device %d out of range", dev);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        if (!check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "output_argmax_noalloc: scratch address", err,
                       err_len))
            return nullptr;
        if (!p) {
            set_err(err, err_len, "output_argmax_noalloc: null scratch address");
            return nullptr;
        }
        g_scratch_ptr[dev] = p;
    }
    return g_scratch_ptr[dev];
}

}  // namespace

extern "C" {

int qw35_hip_output_argmax_noalloc(const qw35_hip_weight* w, const float* x, const float* awq, uint32_t n_batch,
                                   uint32_t* token, float* logit, void* stream, char* err, uintptr_t err_len) {
    if (!check_weight(w, "output_argmax_noalloc", err, err_len) ||
        !check_gemv_type(w, "output_argmax_noalloc", err, err_len) ||
        !check_chunked_k(w, "output_argmax_noalloc", err, err_len))
        return 0;
    if (n_batch < 1 || n_batch > QW35_HIP_MAX_BATCH) {
        set_err(err, err_len, "output_argmax_noalloc: n_batch=%u must be in 1..%u", n_batch, QW35_HIP_MAX_BATCH);
        return 0;
    }
    const uint64_t need = 2 * argmax_ws_part(w, n_batch);
    if (need > QW35_HIP_ARGMAX_SCRATCH_BYTES) {
        set_err(err, err_len,
                "output_argmax_noalloc: the partials of a %llu-row head at batch %u take %llu bytes and exceed the "
                "library's %llu-byte array; use qw35_hip_output_argmax with a workspace",
                (unsigned long long)w->rows, n_batch, (unsigned long long)need,
                (unsigned long long)QW35_HIP_ARGMAX_SCRATCH_BYTES);
        return 0;
    }
    void* ptr = scratch_of_current_device(err, err_len);
    if (!ptr) return 0;
    // Same validation and kernels as the workspace entry point, over the array.
    return qw35_hip_output_argmax(w, x, awq, n_batch, token, logit, ptr, QW35_HIP_ARGMAX_SCRATCH_BYTES, stream, err,
                                  err_len);
}

uint32_t qw35_hip_stream_read_sink_len(uint64_t bytes) { return qw35::stream_read_blocks(bytes); }

int qw35_hip_stream_read(const void* buf, uint64_t bytes, uint32_t* sink, void* stream, char* err,
                         uintptr_t err_len) {
    if (!buf || !sink || bytes == 0) {
        set_err(err, err_len, "stream_read: null buffer or sink, or zero bytes");
        return 0;
    }
    if ((bytes & 15u) || ((uintptr_t)buf & 15u) || ((uintptr_t)sink & 3u)) {
        set_err(err, err_len, "stream_read: buf and bytes must be 16-byte aligned, sink 4-byte aligned");
        return 0;
    }
    return check_hip(qw35::launch_stream_read(buf, bytes, sink, static_cast<hipStream_t>(stream)), "stream_read", err,
                     err_len)
               ? 1
               : 0;
}

int qw35_hip_mfma_probe(uint32_t n_workgroups, uint32_t iters, float* sink, void* stream, char* err,
                        uintptr_t err_len) {
    if (!sink || n_workgroups < 1 || n_workgroups > 65536 || iters < 1 || iters > 1000000) {
        set_err(err, err_len, "mfma_probe: null sink, or n_workgroups outside 1..65536 or iters outside 1..1000000");
        return 0;
    }
    if ((uintptr_t)sink & 3u) {
        set_err(err, err_len, "mfma_probe: sink must be 4-byte aligned");
        return 0;
    }
    return check_hip(qw35::launch_mfma_probe(n_workgroups, iters, sink, static_cast<hipStream_t>(stream)),
                     "mfma_probe", err, err_len)
               ? 1
               : 0;
}

int qw35_hip_sync(void* stream, char* err, uintptr_t err_len) {
    hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    if (e == hipSuccess) e = hipGetLastError();
    return check_hip(e, "sync", err, err_len) ? 1 : 0;
}

}  // extern "C"
