"""The Qwen3.5 decode-step projection sequence: layer layout, tensor names,
shapes, and a recorded plan over synthetic weights.

The layout follows the reference runtime:

* layer kinds: layer ``il`` is gated full attention when
  ``(il + 1) % full_attention_interval == 0`` and Gated DeltaNet ("delta")
  otherwise (qw35-server/src/metal/bridge/Qw35MetalRuntime.m:326-372,
  qw35-server/src/graph.rs:72-91);
* tensor names ``blk.{il}.attn_q.weight`` ... ``output.weight`` and the order
  in which one token's projections run (``encodeDecodeLayers``,
  Qw35MetalRuntime.m:1170-1221): the mixer's input projections over the layer
  input norm (delta: qkv, gate, beta, alpha, Qw35MetalRuntime+SSM.m:22-25;
  attention: q, k, v, Qw35MetalRuntime+Attention.m:35-37), the mixer's output
  projection with the residual add (+SSM.m:56, +Attention.m:113), the FFN
  gate/up/SwiGLU over the post-attention norm and the down projection with the
  residual add (Qw35MetalRuntime+FFN.m:13-35), then the output head
  (Qw35MetalRuntime+Output.m:11-65);
* shapes from the hyper-parameters (``qw35_metal_hparams``,
  qw35-server/src/metal/bridge/Qw35MetalTypes.h:30-59; buffer sizing
  Qw35MetalRuntime.m:377-387): attn_q rows = heads * key_length * (2 if the
  output gate is fused), attn_k / attn_v rows = kv_heads * key / value length,
  attn_output k = heads * value_length, attn_qkv rows = ssm_inner + 2 * groups
  * state, attn_gate rows = ssm_inner, ssm_beta / ssm_alpha rows =
  time_step_rank, ssm_out k = ssm_inner.

Only the projections are run here; the attention, DeltaNet recurrence, norms
and residual adds between them are not part of this library, so the plan reads
its inputs from buffers the caller owns and refreshes.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import runtime as rt


@dataclass(frozen=True)
class Hparams:
    """The projection-relevant fields of ``qw35_metal_hparams`` plus the vocabulary."""

    transformer_layers: int = 32
    embedding_length: int = 4096
    feed_forward_length: int = 12288
    attention_heads: int = 16
    attention_kv_heads: int = 4
    attention_key_length: int = 256
    attention_value_length: int = 256
    ssm_state_size: int = 128
    ssm_group_count: int = 16
    ssm_time_step_rank: int = 32
    ssm_inner_size: int = 4096
    full_attention_interval: int = 4
    attn_gate: int = 1
    vocab: int = 248320


QWEN35_9B = Hparams()


def is_attention_layer(hp: Hparams, il: int) -> bool:
    interval = hp.full_attention_interval or 4
    return (il + 1) % interval == 0


@dataclass(frozen=True)
class Proj:
    """One projection: tensor name suffix, rows, k, and the buffer it reads."""

    name: str
    rows: int
    k: int
    reads: str  # "norm" (layer input norm), "core" (mixer output), "ffn_norm", "ffn_act"


def mixer_projections(hp: Hparams, il: int) -> list[Proj]:
    """Input projections (in dispatch order) and the output projection of layer il's mixer."""
    e = hp.embedding_length
    if is_attention_layer(hp, il):
        q_rows = hp.attention_heads * hp.attention_key_length * (2 if hp.attn_gate else 1)
        kv_k = hp.attention_kv_heads * hp.attention_key_length
        kv_v = hp.attention_kv_heads * hp.attention_value_length
        return [Proj("attn_q", q_rows, e, "norm"), Proj("attn_k", kv_k, e, "norm"), Proj("attn_v", kv_v, e, "norm"),
                Proj("attn_output", e, hp.attention_heads * hp.attention_value_length, "core")]
    qkv = hp.ssm_inner_size + 2 * hp.ssm_group_count * hp.ssm_state_size
    return [Proj("attn_qkv", qkv, e, "norm"), Proj("attn_gate", hp.ssm_inner_size, e, "norm"),
            Proj("ssm_beta", hp.ssm_time_step_rank, e, "norm"), Proj("ssm_alpha", hp.ssm_time_step_rank, e, "norm"),
            Proj("ssm_out", e, hp.ssm_inner_size, "core")]


def ffn_projections(hp: Hparams) -> list[Proj]:
    e, f = hp.embedding_length, hp.feed_forward_length
    return [Proj("ffn_gate", f, e, "ffn_norm"), Proj("ffn_up", f, e, "ffn_norm"), Proj("ffn_down", e, f, "ffn_act")]


def core_width(hp: Hparams, il: int) -> int:
    return mixer_projections(hp, il)[-1].k


def projection_bytes(hp: Hparams, types: "StackTypes") -> int:
    """Weight bytes one decode step streams (every projection once, plus the head)."""
    total = 0
    for il in range(hp.transformer_layers):
        for p in mixer_projections(hp, il):
            total += p.rows * rt.row_bytes(types.mixer, p.k)
        for p in ffn_projections(hp):
            total += p.rows * rt.row_bytes(types.ffn, p.k)
    return total + hp.vocab * rt.row_bytes(types.head, hp.embedding_length)


@dataclass(frozen=True)
class StackTypes:
    """Codec of each projection group (config 5: q8_0 mixers, GF4 FFN, Q4_K head)."""

    mixer: int = rt.TYPE_Q8_0
    ffn: int = rt.TYPE_GF4
    head: int = rt.TYPE_Q4_K


def synthetic_weight(gen: torch.Generator, type_id: int, rows: int, k: int, std: float = 0.02,
                     row_block: int = 32768) -> rt.HipWeight:
    """A rows x k weight encoded on the GPU from N(0, std) (bf16-rounded for GF4,
    as the GF4 configs specify), made ``row_block`` rows at a time."""
    dev = gen.device
    rb = rt.row_bytes(type_id, k)
    raw = torch.empty(rows * rb, dtype=torch.uint8, device=dev)
    for r0 in range(0, rows, row_block):
        n = min(row_block, rows - r0)
        src = torch.randn((n, k), generator=gen, device=dev, dtype=torch.float32) * std
        if type_id == rt.TYPE_GF4:
            src = src.to(torch.bfloat16).to(torch.float32)
        raw[r0 * rb:(r0 + n) * rb].copy_(rt.quantize(src, type_id))
        del src
    return rt.HipWeight.from_device(raw, type_id, rows, k)


@dataclass
class ProjectionStack:
    """Synthetic weights of every projection of a Qwen3.5 decode step.

    ``layers[il]`` maps a tensor-name suffix (``attn_q``, ``ffn_down``, ...) to
    its ``HipWeight``; ``head`` is ``output.weight``.  ``distinct`` makes every
    layer's weights different (tests); otherwise each shape is encoded once and
    its bytes copied into every layer's own buffer (same bytes streamed, less
    set-up time: the benchmark).
    """

    hp: Hparams
    types: StackTypes
    layers: list[dict[str, rt.HipWeight]]
    head: rt.HipWeight

    @classmethod
    def synthetic(cls, hp: Hparams = QWEN35_9B, types: StackTypes = StackTypes(), seed: int = 1,
                  distinct: bool = True, head_tile_rows: int | None = None,
                  device: str | torch.device = "cuda") -> "ProjectionStack":
        gen = torch.Generator(device=device)
        gen.manual_seed(seed)
        cache: dict[tuple, rt.HipWeight] = {}

        def make(type_id, rows, k):
            if distinct:
                return synthetic_weight(gen, type_id, rows, k)
            key = (type_id, rows, k)
            if key not in cache:
                cache[key] = synthetic_weight(gen, type_id, rows, k)
            base = cache[key]
            return rt.HipWeight.from_device(base.storage.clone(), type_id, rows, k)

        layers = []
        for il in range(hp.transformer_layers):
            ws = {p.name: make(types.mixer, p.rows, p.k) for p in mixer_projections(hp, il)}
            ws.update({p.name: make(types.ffn, p.rows, p.k) for p in ffn_projections(hp)})
            layers.append(ws)
        cache.clear()
        if head_tile_rows is None or head_tile_rows >= hp.vocab:
            head = synthetic_weight(gen, types.head, hp.vocab, hp.embedding_length)
        else:  # repeat a block of distinct rows (the benchmark: same bytes, less set-up)
            part = synthetic_weight(gen, types.head, head_tile_rows, hp.embedding_length)
            rb = rt.row_bytes(types.head, hp.embedding_length)
            full = torch.empty(hp.vocab * rb, dtype=torch.uint8, device=part.storage.device)
            for r0 in range(0, hp.vocab, head_tile_rows):
                n = min(head_tile_rows, hp.vocab - r0)
                full[r0 * rb:(r0 + n) * rb].copy_(part.storage[:n * rb])
            head = rt.HipWeight.from_device(full, types.head, hp.vocab, hp.embedding_length)
        return cls(hp, types, layers, head)

    @property
    def weight_bytes(self) -> int:
        return sum(w.storage.numel() for ws in self.layers for w in ws.values()) + self.head.storage.numel()


@dataclass
class StepBuffers:
    """Device buffers one decode step's projections read and write.

    Inputs (the caller refreshes them in place): ``norm`` (layer input norm),
    ``core`` (mixer output, per width), ``ffn_norm`` (post-attention norm) and
    ``awq`` (the FFN's per-input-channel scale, or None).  Outputs:
    ``mixer_out[il][name]`` (each input projection of each layer), ``ffn_act[il]``
    (SwiGLU output, read by that layer's down projection), ``act`` (the residual
    stream: every output and down projection adds into it) and ``logits``.
    ``shared_outputs`` reuses one set of mixer / FFN output buffers for every
    layer, as the reference runtime does (the benchmark); otherwise every layer
    has its own, so that each output can be checked (the tests).
    """

    norm: torch.Tensor
    core: dict[int, torch.Tensor]
    ffn_norm: torch.Tensor
    awq: torch.Tensor | None
    act: torch.Tensor
    mixer_out: list[dict[str, torch.Tensor]]
    ffn_act: list[torch.Tensor]
    logits: torch.Tensor

    @classmethod
    def make(cls, hp: Hparams, n_batch: int, gen: torch.Generator, awq: bool = True,
             shared_outputs: bool = False) -> "StepBuffers":
        dev = gen.device
        e = hp.embedding_length

        def normal(*shape):
            return torch.randn(shape, generator=gen, device=dev, dtype=torch.float32)

        widths = sorted({core_width(hp, il) for il in range(hp.transformer_layers)})
        core = {w: normal(n_batch, w) for w in widths}
        a = (torch.rand((e,), generator=gen, device=dev) * 1.5 + 0.5) if awq else None
        outs, acts = [], []
        shared_mix: dict[str, torch.Tensor] = {}
        shared_act = None
        for il in range(hp.transformer_layers):
            d = {}
            for p in mixer_projections(hp, il)[:-1]:
                if shared_outputs:
                    d[p.name] = shared_mix.setdefault(
                        p.name, torch.zeros((n_batch, p.rows), dtype=torch.float32, device=dev))
                else:
                    d[p.name] = torch.zeros((n_batch, p.rows), dtype=torch.float32, device=dev)
            outs.append(d)
            if shared_outputs:
                if shared_act is None:
                    shared_act = torch.zeros((n_batch, hp.feed_forward_length), dtype=torch.float32, device=dev)
                acts.append(shared_act)
            else:
                acts.append(torch.zeros((n_batch, hp.feed_forward_length), dtype=torch.float32, device=dev))
        return cls(norm=normal(n_batch, e), core=core, ffn_norm=normal(n_batch, e), awq=a,
                   act=normal(n_batch, e), mixer_out=outs, ffn_act=acts,
                   logits=torch.zeros((n_batch, hp.vocab), dtype=torch.float32, device=dev))


def build_plan(stack: ProjectionStack, bufs: StepBuffers, head: bool = True) -> rt.DecodePlan:
    """Record one decode step's projections, in the reference's dispatch order,
    as a ``DecodePlan``: per layer the mixer input projections (merged into one
    launch where they share the input), the output projection (+= into ``act``),
    the fused gate/up/SwiGLU and the down projection (+= into ``act``); then the
    head into ``logits``."""
    hp = stack.hp
    plan = rt.DecodePlan()
    for il, ws in enumerate(stack.layers):
        mix = mixer_projections(hp, il)
        for p in mix[:-1]:
            plan.matvec(ws[p.name], bufs.norm, bufs.mixer_out[il][p.name])
        out = mix[-1]
        plan.matvec(ws[out.name], bufs.core[out.k], bufs.act, residual=True)
        plan.swiglu(ws["ffn_gate"], ws["ffn_up"], bufs.ffn_norm, bufs.ffn_act[il], awq=bufs.awq)
        plan.matvec(ws["ffn_down"], bufs.ffn_act[il], bufs.act, residual=True)
    if head:
        plan.matvec(stack.head, bufs.norm, bufs.logits)
    return plan.record()


def chunk_workspace(stack: ProjectionStack, n_tokens: int, device=None) -> torch.Tensor:
    """A prefill workspace that holds every projection's planned launch at n_tokens
    (fp32 activations), as the projection runtime sizes its own."""
    import ctypes as C

    from . import _ffi

    lib = _ffi.load()
    size = max(int(lib.qw35_hip_matmul_prefill_workspace_size(C.byref(w.prefill.view), n_tokens))
               for ws in stack.layers for w in ws.values())
    # a layer's mixer input projections of one weight form run as one launch
    # over their summed rows (the plan merges them): size that launch too
    for il, ws in enumerate(stack.layers):
        views = [ws[p.name].prefill.view for p in mixer_projections(stack.hp, il)[:-1]]
        i = 0
        while i < len(views):
            merged = _ffi.Weight.from_buffer_copy(views[i])
            j = i + 1
            while (j < len(views) and j - i < 4 and merged.rows % 4 == 0 and views[j].type_id == merged.type_id
                   and views[j].k == merged.k and views[j].rows % 4 == 0):
                merged.rows += views[j].rows
                merged.bytes += views[j].bytes
                j += 1
            if j - i > 1:
                size = max(size, int(lib.qw35_hip_matmul_prefill_workspace_size(C.byref(merged), n_tokens)))
            i = j
    return torch.empty(size, dtype=torch.uint8, device=device or stack.head.storage.device)


def build_chunk_plan(stack: ProjectionStack, bufs: StepBuffers, workspace: torch.Tensor,
                     head: bool = True) -> rt.DecodePlan:
    """Record one prefill chunk's projections (the projection part of
    ``evalTokens``, Qw35MetalRuntime.m:1227-1333) over the n rows of ``bufs``
    (fp32 activations, n > 8): per layer the mixer input projections, the
    output projection added into ``act``, gate/up/SwiGLU (the up projection's
    SwiGLU epilogue) and the down projection added into ``act``, all on the
    prefill matmul; then the head on the last token's norm row as a GEMV into
    ``logits[0]`` -- the sequence ``qw35_hip_runtime_eval_chunk`` records."""
    hp = stack.hp
    plan = rt.DecodePlan()
    for il, ws in enumerate(stack.layers):
        mix = mixer_projections(hp, il)
        for p in mix[:-1]:
            plan.matmul(ws[p.name], bufs.norm, bufs.mixer_out[il][p.name], workspace)
        out = mix[-1]
        plan.matmul(ws[out.name], bufs.core[out.k], bufs.act, workspace, residual=True)
        plan.matmul_swiglu(ws["ffn_gate"], ws["ffn_up"], bufs.ffn_norm, bufs.ffn_act[il], workspace, awq=bufs.awq)
        plan.matmul(ws["ffn_down"], bufs.ffn_act[il], bufs.act, workspace, residual=True)
    if head:
        n = bufs.norm.shape[0]
        plan.matvec(stack.head, bufs.norm[n - 1:n], bufs.logits[0:1])
    return plan.record()


def chunk_flops(hp: Hparams, n_tokens: int) -> float:
    """Multiply-add flops of a chunk's projections (2 n rows k per projection; the head not counted)."""
    per_token = sum(p.rows * p.k for il in range(hp.transformer_layers) for p in mixer_projections(hp, il))
    per_token += hp.transformer_layers * sum(p.rows * p.k for p in ffn_projections(hp))
    return 2.0 * n_tokens * per_token


def gemv_count(hp: Hparams, head: bool = True) -> int:
    """GEMVs of one step as the reference dispatches them (fused gate/up counts once)."""
    n = sum(len(mixer_projections(hp, il)) + 2 for il in range(hp.transformer_layers))
    return n + (1 if head else 0)


def gguf_name(il: int | None, proj: str) -> str:
    """GGUF tensor name of a projection: ``blk.{il}.{proj}.weight``, or ``output.weight`` (il None)."""
    return "output.weight" if il is None else f"blk.{il}.{proj}.weight"


def stack_tensors(stack: ProjectionStack) -> list[tuple[str, tuple[int, int], int, torch.Tensor]]:
    """(GGUF name, dims (k, rows), type id, device bytes) of every projection of a stack, in layer order."""
    out = []
    for il, ws in enumerate(stack.layers):
        for name, w in ws.items():
            out.append((gguf_name(il, name), (w.k, w.rows), w.type_id, w.storage))
    h = stack.head
    out.append((gguf_name(None, "output"), (h.k, h.rows), h.type_id, h.storage))
    return out
