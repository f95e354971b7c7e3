"""A Qwen2 runner with swappable kernels: the consumer the hot path is a drop-in for.

Public surface of the reference's kernels/e2e/model.py: `Linear`, `Backend`, `W4RefBackend`,
`OursBackend`, `OursFP8Backend`, `make_backend(name)`, `QwenRunner(hf_model, backend, max_len,
batch)`, `QwenRunner.forward(tokens, pos, all_logits)`, `QwenRunner.weight_bytes()`. Inside it is
laid out for one MI355X:

- A backend is a weight format plus the ops over it. `Backend.pack(w, b)` turns an fp16 [N, K]
  weight into the backend's `Linear` (fp16, int4 RTN or OCP e4m3); `linear`, `norm`, `act` and
  their fused pairs (`norm_linear`, `linear_norm_linear`, `act_linear`) are what differs between
  runs. Embedding, RoPE, attention and the tied fp16 lm_head are the same code for every backend.
- The lm_head and final norm are chosen by the runner, not the backend (`head=`), so every
  backend runs the same head: "gemv" streams the fp16 table through this build's one-row GEMV
  (with the final RMSNorm in the same launch) at decode rows, "torch" keeps
  `F.linear(h, lm_head)` after the norm as the reference does (model.py:250-253). A `_lm`
  backend instead quantizes a copy of the table in its own format.
- q/k/v and gate/up are concatenated into one projection each (model.py:168-191).
- The KV cache is kept in the fused decode attention's tiled operand order (K tiles and V^T
  tiles, kernels/attention.py), max_len a multiple of 32. The torch path (prompt steps) writes
  it with kernels.attention.write_kv and reads K and V back in the reference's [.., max_len,
  head_dim] order.
- Every step is capturable in a hipGraph: positions are device tensors, the cache is written
  by index on device, the causal mask is built from the positions inside the graph.

The model comes from a Hugging Face Qwen2 module object (as in the reference) or from
`random_qwen2`, which builds the Qwen2.5-1.5B architecture with Hugging Face's initialisation
(linear and embedding weights N(0, 0.02), biases 0, norm weights 1) on the GPU, seeded, with no
download.
"""

from __future__ import annotations

from dataclasses import dataclass, fields

import torch
import torch.nn.functional as F

from kernels import config


# ----------------------------------------------------------------------------------- backends
@dataclass
class Linear:
    """One projection (model.py:25-33): fp16 `w`, or the packed tensors of a quantized format
    (int4: qweight/scales/zeros; e4m3: qweight = wq [K, N], scales = per-channel scale)."""

    w: torch.Tensor | None = None
    qweight: torch.Tensor | None = None
    scales: torch.Tensor | None = None
    zeros: torch.Tensor | None = None
    bias: torch.Tensor | None = None

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (getattr(self, f.name) for f in fields(self))
                   if t is not None)


def _rmsnorm_torch(x, w, eps, residual=None):
    """Qwen2 RMSNorm with HF rounding steps in torch ops (the fp16 side of the comparison):
    fp16 residual add, fp32 mean of squares, fp16 normalized value, multiply by w."""
    if residual is not None:
        x = x + residual
    h = x.float()
    normed = (h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype)
    out = w * normed
    return out if residual is None else (out, x)


class Backend:
    """fp16 weights, eager torch ops (hipBLASLt GEMMs), HF Qwen2 numerics (model.py:36-52)."""

    name = "fp16"
    quantized = False
    merges_attention = False  # attn_linear_norm_linear takes the attention's range partials
    fuses_prompt_act = False  # linear_norm_linear_act forms the activation in gate_up (prompt rows)
    # the fused attention's launch warms the next weights (QwenRunner.warm_set): fp16 254 -> 259
    # tok/s, W4A16 1305 -> 1361 (e2e, one MI355X)
    warms = True
    quant_lm_head = False

    def pack(self, w: torch.Tensor, b: torch.Tensor | None) -> Linear:
        """The backend's stored form of an fp16 [N, K] weight and its bias."""
        return Linear(w=w, bias=b)

    def linear(self, x, p: Linear):
        return F.linear(x, p.w, p.bias)

    def norm(self, x, w, eps, residual=None):
        return _rmsnorm_torch(x, w, eps, residual)

    def act(self, gate_up):
        gate, up = gate_up.chunk(2, dim=-1)
        return F.silu(gate) * up

    def norm_linear(self, x, w, eps, residual, p: Linear):
        """norm then linear, the order of the reference's layer (model.py:226-233): returns the
        projection of the normalized row and the updated residual (None without one)."""
        if residual is None:
            return self.linear(self.norm(x, w, eps), p), None
        h, res = self.norm(x, w, eps, residual=residual)
        return self.linear(h, p), res

    def act_linear(self, gate_up, p: Linear):
        """act then linear (the MLP's down projection, model.py:233)."""
        return self.linear(self.act(gate_up), p)

    def linear_norm_linear(self, x, p1: Linear, residual, w, eps, p2: Linear):
        """linear, then norm (+ residual) then linear: the attention output projection, the
        post-attention norm and gate_up (model.py:226-233). Returns (y2, new residual)."""
        return self.norm_linear(self.linear(x, p1), w, eps, residual, p2)

    def linear_norm_linear_act(self, x, p1: Linear, residual, w, eps, p2: Linear):
        """linear_norm_linear, then the activation of its gate_up output (model.py:226-234).
        Returns (act, new residual)."""
        y2, res = self.linear_norm_linear(x, p1, residual, w, eps, p2)
        return self.act(y2), res


class _Int4:
    """The int4 RTN format of kernels.quant (group 128, packed [K/8, N], fp16 scales/zeros)."""

    quantized = True

    def pack(self, w, b) -> Linear:
        from kernels.quant import quantize_rtn

        qw, s, z = quantize_rtn(w, config.GROUP_SIZE)
        return Linear(qweight=qw, scales=s, zeros=z, bias=b)


class W4RefBackend(_Int4, Backend):
    """RTN int4 weights dequantized once (bit-exact HIP dequantizer) then the fp16 GEMM: the same
    quantized model as `ours` through library GEMMs (model.py:55-67)."""

    name = "w4_ref"
    warms = False  # its GEMMs read the dequantized fp16 copy, not the packed weights warm_set names

    def linear(self, x, p: Linear):
        if p.w is None:
            from kernels.quant import dequantize

            p.w = dequantize(p.qweight, p.scales, p.zeros, config.GROUP_SIZE)
        return F.linear(x, p.w, p.bias)


class FP8RefBackend(Backend):
    """OCP e4m3 weights with per-channel scales (kernels.fp8.quantize_fp8), dequantized once to
    fp16 (bit-exact HIP dequantizer, fp8.py:33-35) then the fp16 GEMM: the same quantized model
    as `ours_fp8` through library GEMMs, the FP8 counterpart of `w4_ref`."""

    name = "fp8_ref"
    quantized = True
    warms = False  # its GEMMs read the dequantized fp16 copy

    def pack(self, w, b) -> Linear:
        from kernels.fp8 import quantize_fp8

        wq, per_channel = quantize_fp8(w)
        return Linear(qweight=wq, scales=per_channel, bias=b)

    def linear(self, x, p: Linear):
        if p.w is None:
            from kernels.fp8 import dequantize_fp8

            p.w = dequantize_fp8(p.qweight, p.scales)
        return F.linear(x, p.w, p.bias)


class OursBackend(_Int4, Backend):
    """This build's kernels: W4A16 GEMV/GEMM, fused RMSNorm+residual, fused SwiGLU
    (model.py:70-97).

    entry="matmul" (`ours`) sends every projection through `w4a16_matmul` and, at one decode
    row, fuses the norm and activation launches into the projections (kernels.fused).
    entry="decode" (`ours_cuda`, the reference's name for its native decode kernel) sends rows
    <= 16 through `kernels.cuda.w4a16_cuda.w4a16_decode_cuda` and runs norm and activation as
    launches of their own, as the reference's `ours_cuda` does."""

    def __init__(self, entry: str = "matmul"):
        if entry not in ("matmul", "decode"):
            raise ValueError(f"OursBackend: entry {entry!r}, expected 'matmul' or 'decode'")
        self.entry = entry
        self.name = "ours" if entry == "matmul" else "ours_cuda"

    @property
    def fused(self) -> bool:
        return self.entry == "matmul"

    def linear(self, x, p: Linear):
        if self.entry == "decode" and x.numel() <= 16 * x.shape[-1]:
            from kernels.cuda.w4a16_cuda import w4a16_decode_cuda

            return w4a16_decode_cuda(x, p.qweight, p.scales, p.zeros, bias=p.bias)
        from kernels.w4a16 import w4a16_matmul

        return w4a16_matmul(x, p.qweight, p.scales, p.zeros, bias=p.bias)

    def norm(self, x, w, eps, residual=None):
        from kernels.rmsnorm import rmsnorm

        return rmsnorm(x, w, eps, residual)

    def act(self, gate_up):
        from kernels.swiglu import swiglu_fused

        return swiglu_fused(gate_up)

    def norm_linear(self, x, w, eps, residual, p: Linear):
        """One launch at decode: the RMSNorm (+ residual) forms the activation inside the W4A16
        kernel's x staging (kernels.fused)."""
        if not self.fused:
            return super().norm_linear(x, w, eps, residual, p)
        from kernels.fused import rmsnorm_w4a16_matmul

        return rmsnorm_w4a16_matmul(x, w, eps, residual, p.qweight, p.scales, p.zeros,
                                    config.GROUP_SIZE, p.bias)

    @property
    def merges_attention(self) -> bool:
        return self.fused

    def attn_linear_norm_linear(self, ranges, p1: Linear, residual, w, eps, p2: Linear):
        """linear_norm_linear with x the decode attention left as range partials
        (kernels.attention.decode_attention_ranges): the o projection merges the ranges while it
        stages x, so the attention's merge and the projection are one launch
        (kernels.fused.attn_linear_rmsnorm_w4a16_matmul)."""
        from kernels.fused import attn_linear_rmsnorm_w4a16_matmul

        return attn_linear_rmsnorm_w4a16_matmul(ranges, p1.qweight, p1.scales, p1.zeros, p1.bias,
                                                residual, w, eps, p2.qweight, p2.scales, p2.zeros,
                                                p2.bias, config.GROUP_SIZE)

    def linear_norm_linear(self, x, p1: Linear, residual, w, eps, p2: Linear):
        """Two launches at decode: the first projection's epilogue adds the residual and
        publishes the row's partial sums of squares, the second forms the norm while it stages
        its input (kernels.fused.linear_rmsnorm_w4a16_matmul)."""
        if not self.fused:
            return super().linear_norm_linear(x, p1, residual, w, eps, p2)
        from kernels.fused import linear_rmsnorm_w4a16_matmul

        return linear_rmsnorm_w4a16_matmul(x, p1.qweight, p1.scales, p1.zeros, p1.bias, residual,
                                           w, eps, p2.qweight, p2.scales, p2.zeros, p2.bias,
                                           config.GROUP_SIZE)

    @property
    def fuses_prompt_act(self) -> bool:
        return self.fused

    def linear_norm_linear_act(self, x, p1: Linear, residual, w, eps, p2: Linear):
        """Prompt rows: the o projection, the post-attention norm with the residual, then gate_up
        with SwiGLU in the prefill GEMM's epilogue (kernels.fused.w4a16_matmul_swiglu: the same
        bits as gate_up then SwiGLU, one launch and no [T, 2I] intermediate where the plan is the
        prefill GEMM). Returns (act, new residual)."""
        from kernels.fused import w4a16_matmul_swiglu

        h, res = self.norm(self.linear(x, p1), w, eps, residual=residual)
        return w4a16_matmul_swiglu(h, p2.qweight, p2.scales, p2.zeros, config.GROUP_SIZE, p2.bias), res

    def act_linear(self, gate_up, p: Linear):
        """One launch at decode: SwiGLU forms the down projection's activation (kernels.fused)."""
        if not self.fused:
            return super().act_linear(gate_up, p)
        from kernels.fused import swiglu_w4a16_matmul

        return swiglu_w4a16_matmul(gate_up, p.qweight, p.scales, p.zeros, config.GROUP_SIZE,
                                   p.bias)


class OursFP8Backend(OursBackend):
    """FP8 (OCP e4m3) weight-only linears with the same fused norm and activation
    (model.py:100-118). `Linear.qweight` holds wq [K, N], `Linear.scales` the per-channel
    scale."""

    warms = False  # twice the int4 bytes: warming them measured slower (1105 -> 1042 tok/s)

    def __init__(self):
        super().__init__("matmul")
        self.name = "ours_fp8"

    def quantize(self, w, b) -> Linear:
        """e4m3 weights [K, N] with per-channel scales. `quantize` is the hook the reference's
        runner looks for on formats other than int4 RTN (model.py:109-112,175-176), so this
        backend also packs its weights correctly under that runner; this runner calls `pack`."""
        from kernels.fp8 import quantize_fp8

        wq, per_channel = quantize_fp8(w)
        return Linear(qweight=wq, scales=per_channel, bias=b)

    pack = quantize

    def linear(self, x, p: Linear):
        from kernels.fp8 import w8a16_matmul

        return w8a16_matmul(x, p.qweight, p.scales, bias=p.bias)

    def norm_linear(self, x, w, eps, residual, p: Linear):
        """One launch at decode: the RMSNorm (+ residual) forms the FP8 projection's activation
        (kernels.fused.rmsnorm_w8a16_matmul)."""
        from kernels.fused import rmsnorm_w8a16_matmul

        return rmsnorm_w8a16_matmul(x, w, eps, residual, p.qweight, p.scales, bias=p.bias)

    linear_norm_linear = Backend.linear_norm_linear  # the residual-statistics pair is W4A16

    def linear_norm_linear_act(self, x, p1: Linear, residual, w, eps, p2: Linear):
        """Prompt rows: the o projection, the post-attention norm with the residual, then gate_up
        with SwiGLU in the e4m3 prefill GEMM's epilogue (kernels.fused.w8a16_matmul_swiglu, the
        same bits as gate_up then SwiGLU). Returns (act, new residual)."""
        from kernels.fused import w8a16_matmul_swiglu

        h, res = self.norm(self.linear(x, p1), w, eps, residual=residual)
        return w8a16_matmul_swiglu(h, p2.qweight, p2.scales, bias=p2.bias), res

    def attn_linear_norm_linear(self, ranges, p1: Linear, residual, w, eps, p2: Linear):
        """linear_norm_linear with x the decode attention left as range partials: the FP8 o
        projection merges the ranges in its x staging (kernels.fused.attn_w8a16_matmul), then the
        residual + RMSNorm forms gate_up's activation (kernels.fused.rmsnorm_w8a16_matmul)."""
        from kernels.fused import attn_w8a16_matmul, rmsnorm_w8a16_matmul

        y = attn_w8a16_matmul(ranges, p1.qweight, p1.scales, p1.bias).view(residual.shape)
        return rmsnorm_w8a16_matmul(y, w, eps, residual, p2.qweight, p2.scales, bias=p2.bias)

    def act_linear(self, gate_up, p: Linear):
        """One launch at decode: SwiGLU forms the FP8 down projection's activation
        (kernels.fused.swiglu_w8a16_matmul)."""
        from kernels.fused import swiglu_w8a16_matmul

        return swiglu_w8a16_matmul(gate_up, p.qweight, p.scales, bias=p.bias)


# name -> factory. `<name>_lm` is `<name>` with the lm_head quantized in its format too
# (model.py:121-136); only quantized formats take it.
BACKENDS = {
    "fp16": Backend,
    "w4_ref": W4RefBackend,
    "ours": OursBackend,
    "ours_cuda": lambda: OursBackend("decode"),
    "ours_fp8": OursFP8Backend,
    "fp8_ref": FP8RefBackend,
}


def make_backend(name: str) -> Backend:
    """The backend registered as `name`; a trailing `_lm` asks for the lm_head in the backend's
    own weight format as well (model.py:121-136), which only the quantizing backends offer."""
    head_too = name.endswith("_lm")
    base = name[: len(name) - 3] if head_too else name
    factory = BACKENDS.get(base)
    if factory is None:
        raise KeyError(f"unknown backend {name!r}; known: {sorted(BACKENDS)} (+ '_lm')")
    backend = factory()
    if head_too and not backend.quantized:
        raise ValueError(f"{name}: backend {base!r} keeps fp16 weights and has no format to put "
                         "lm_head in")
    if head_too:
        backend.name = name
    backend.quant_lm_head = head_too
    return backend


# -------------------------------------------------------------------------------------- model
def qwen25_15b_config(**overrides):
    """The Qwen2.5-1.5B architecture as a transformers Qwen2Config (no weights)."""
    import transformers

    kw = dict(config.QWEN25_15B)
    kw.update(overrides)
    theta = kw.pop("rope_theta")
    kw.pop("head_dim", None)
    return transformers.Qwen2Config(**kw, rope_theta=theta, max_position_embeddings=32768)


def random_qwen2(cfg=None, seed: int = 4, device="cuda", dtype=torch.float16):
    """A random-init Qwen2ForCausalLM (HF initialisation) built directly on `device`."""
    import transformers

    cfg = cfg or qwen25_15b_config()
    torch.manual_seed(seed)
    if device != "cpu":
        torch.cuda.manual_seed(seed)
    with torch.device(device):
        model = transformers.Qwen2ForCausalLM(cfg)
    return model.to(dtype).eval()


@dataclass
class Arch:
    """What the forward needs from a Qwen2 config."""

    n_heads: int
    n_kv: int
    head_dim: int
    eps: float
    rope_theta: float

    @classmethod
    def of(cls, cfg) -> "Arch":
        head_dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
        rope = getattr(cfg, "rope_parameters", None) or {}
        theta = rope.get("rope_theta", getattr(cfg, "rope_theta", 10000.0))
        return cls(cfg.num_attention_heads, cfg.num_key_value_heads, head_dim, cfg.rms_norm_eps,
                   float(theta))


@dataclass
class Layer:
    ln1: torch.Tensor
    ln2: torch.Tensor
    qkv: Linear
    o: Linear
    gate_up: Linear
    down: Linear


def _concat(*modules):
    """One projection from several nn.Linear modules stacked along the output dimension."""
    w = torch.cat([m.weight.data for m in modules])
    biases = [m.bias for m in modules]
    b = None if biases[0] is None else torch.cat([x.data for x in biases])
    return w, b


class QwenRunner:
    """Static-cache Qwen2 forward with swappable kernels (model.py:150-253)."""

    HEADS = ("gemv", "torch")

    def __init__(self, hf_model, backend: Backend, max_len: int = 2048, batch: int = 1,
                 attention: str = "fused", head: str = "gemv"):
        """attention: "fused" runs decode steps (one token, batch 1) through the fused HIP
        attention kernel (RoPE + KV write + GQA softmax attention in one launch per layer) on
        every backend; "torch" keeps the torch ops for every step. Prefill always uses torch.
        head: "gemv" or "torch", the fp16 lm_head path of every backend (module docstring)."""
        if attention not in ("fused", "torch"):
            raise ValueError(f"attention={attention!r}: 'fused' or 'torch'")
        if head not in self.HEADS:
            raise ValueError(f"head={head!r}: one of {self.HEADS}")
        self.backend = backend
        arch = Arch.of(hf_model.config)
        self.arch = arch
        self.n_heads, self.n_kv, self.head_dim, self.eps = arch.n_heads, arch.n_kv, arch.head_dim, arch.eps
        self.max_len = max_len
        self.head_mode = head
        body = hf_model.model
        self.embed = body.embed_tokens.weight.data
        self.lm_head = hf_model.lm_head.weight.data
        self.final_norm = body.norm.weight.data
        dev, dt = self.embed.device, self.embed.dtype
        d = arch.head_dim
        # HF's rotary frequencies, same expression so the fp32 values agree bit for bit
        self.inv_freq = 1.0 / (arch.rope_theta ** (torch.arange(0, d, 2, device=dev, dtype=torch.float) / d))

        self.layers = [
            Layer(ln1=blk.input_layernorm.weight.data, ln2=blk.post_attention_layernorm.weight.data,
                  qkv=backend.pack(*_concat(blk.self_attn.q_proj, blk.self_attn.k_proj, blk.self_attn.v_proj)),
                  o=backend.pack(*_concat(blk.self_attn.o_proj)),
                  gate_up=backend.pack(*_concat(blk.mlp.gate_proj, blk.mlp.up_proj)),
                  down=backend.pack(*_concat(blk.mlp.down_proj)))
            for blk in body.layers
        ]
        # a `_lm` backend's own copy of the head (the fp16 table stays for the embedding)
        self.head_q = backend.pack(*_concat(hf_model.lm_head)) if backend.quant_lm_head else None

        # K and V^T in the fused attention kernel's tiled operand order (kernels/attention.py);
        # the torch path reads and writes them through the same layout helpers
        from kernels import attention as fa

        if max_len % fa.CHUNK:
            raise ValueError(f"max_len={max_len} must be a multiple of {fa.CHUNK}")
        if d % 32:
            raise ValueError(f"head_dim={d} must be a multiple of 32")
        n = len(self.layers)
        self.k_cache = torch.zeros((n, batch) + fa.k_cache_shape(self.n_kv, max_len, d), device=dev, dtype=dt)
        self.vt_cache = torch.zeros((n, batch) + fa.vt_cache_shape(self.n_kv, max_len, d), device=dev, dtype=dt)
        self.keys = torch.arange(max_len, device=dev)
        self.merge_attention = True  # see forward: the o projection merges the attention's ranges
        self.fuse_prompt_act = True  # see forward: SwiGLU in the prompt's gate_up GEMM
        self.warm_weights = True  # see warm_set: the attention launch warms the next weights
        self.fused_attention = (attention == "fused" and dev.type == "cuda"
                                and fa.supported(d, max_len, batch, 1))
        # prompt rows (T > 1) through kernels.attention.prefill_attention with the fused runner
        self.fused_prefill = (attention == "fused" and dev.type == "cuda" and dt == torch.float16
                              and fa.prefill_supported(d, max_len, batch, 2))

    def weight_bytes(self) -> dict:
        """Bytes of the swapped layers and of the parts that stay fp16 (model.py:196-210). A
        quantized Linear is counted in its stored format (w4_ref's cached fp16 copy excluded)."""
        quantized = self.backend.quantized

        def stored(p: Linear) -> int:
            cached = p.w.nbytes if (quantized and p.w is not None) else 0
            return p.nbytes() - cached

        layers = sum(stored(p) for L in self.layers for p in (L.qkv, L.o, L.gate_up, L.down))
        return {
            "linear_layers": layers,
            "embed": self.embed.nbytes,
            "lm_head_read": stored(self.head_q) if self.head_q is not None else self.lm_head.nbytes,
            "lm_head_quantized": self.head_q is not None,
            "lm_head_shared_with_embed": self.lm_head.data_ptr() == self.embed.data_ptr(),
            "kv_cache": self.k_cache.nbytes + self.vt_cache.nbytes,
        }

    def warm_set(self, i: int) -> list:
        """What the fused decode attention of layer i reads into the caches with its spare
        workgroups (kernels.attention.decode_attention_ranges / decode_attention) while its few
        workgroups run: the weights of the o and gate_up projections after it, their scales and
        zeros, and the next layer's qkv weight (at most 8 ranges). The down projection's weight
        is left out: the warming then ends earlier than down's own reads gain from it."""
        def main(p: Linear):
            return p.qweight if p.qweight is not None else p.w

        L = self.layers[i]
        ts = [main(L.o), main(L.gate_up), L.o.scales, L.o.zeros, L.gate_up.scales, L.gate_up.zeros]
        if i + 1 < len(self.layers):
            ts.append(main(self.layers[i + 1].qkv))
        return [t for t in ts if t is not None]

    def _rope(self, x, cos, sin):
        half = self.head_dim // 2
        return x * cos + torch.cat((-x[..., half:], x[..., :half]), dim=-1) * sin

    def _attend(self, i, q, k, v, pos):
        """q [B, T, nq, hd], k/v [B, T, nkv, hd] (RoPE applied): writes the cache at `pos` and
        returns the attention output [B, T, nq*hd]."""
        B, T = q.shape[:2]
        nkv, hd = self.n_kv, self.head_dim
        g = self.n_heads // nkv
        from kernels import attention as fa

        fa.write_kv(self.k_cache[i], self.vt_cache[i], pos, k.transpose(1, 2), v.transpose(1, 2))
        kc = fa.k_from_tiles(self.k_cache[i])  # [B, nkv, max_len, hd]
        vc = fa.v_from_tiles(self.vt_cache[i])
        # rows ordered (query head within the group, token): [B, nkv, g*T, hd]
        qg = q.view(B, T, nkv, g, hd).permute(0, 2, 3, 1, 4).reshape(B, nkv, g * T, hd)
        scores = torch.matmul(qg, kc.transpose(-1, -2).contiguous()).float() * (hd ** -0.5)
        allowed = self.keys[None, :] <= pos[:, None]  # [T, max_len]
        scores = scores.masked_fill(~allowed.repeat(g, 1), float("-inf"))
        p = torch.softmax(scores, dim=-1).to(q.dtype)
        out = torch.matmul(p, vc)  # [B, nkv, g*T, hd]
        return out.view(B, nkv, g, T, hd).permute(0, 3, 1, 2, 4).reshape(B, T, nkv * g * hd)

    def _logits(self, h, residual):
        """Final norm (+ residual) and lm_head of the last layer's output (model.py:250-253)."""
        be, eps = self.backend, self.eps
        if self.head_q is not None:
            return be.norm_linear(h, self.final_norm, eps, residual, self.head_q)[0]
        if self.head_mode == "gemv":
            from kernels import head as head_mod

            if head_mod.applies(h, self.lm_head) and residual.numel() == h.numel():
                return head_mod.lm_head(h, self.lm_head, norm_weight=self.final_norm, eps=eps,
                                        residual=residual)
        x, _ = be.norm(h, self.final_norm, eps, residual=residual)
        return F.linear(x, self.lm_head)

    @torch.no_grad()
    def forward(self, tokens: torch.Tensor, pos: torch.Tensor, all_logits: bool = False):
        """tokens [B, T]; pos int64 [T] absolute positions. Graph-capturable (model.py:217-253)."""
        be, eps = self.backend, self.eps
        B, T = tokens.shape
        nq, nkv, hd = self.n_heads, self.n_kv, self.head_dim
        x = F.embedding(tokens, self.embed)
        fused = self.fused_attention and B == 1 and T == 1
        prompt = self.fused_prefill and B == 1 and T > 1
        # the attention's ranges merged in the o projection's x staging (one launch fewer per
        # layer, and ranges of a quarter of the cache instead of one range per kv head)
        merge = fused and self.merge_attention and be.merges_attention
        if merge:
            from kernels.attention import MERGE_MAX_RANGES, decode_attention_ranges, ranges_len

            rlen = ranges_len(self.max_len)
            merge = -(-self.max_len // rlen) <= MERGE_MAX_RANGES and config.GROUP_SIZE == 128
        if fused:
            from kernels.attention import decode_attention
        elif prompt:
            from kernels.attention import prefill_attention
        else:
            freqs = pos[:, None].float() * self.inv_freq[None, :]
            emb = torch.cat((freqs, freqs), dim=-1)
            cos = emb.cos().to(x.dtype)[None, :, None, :]
            sin = emb.sin().to(x.dtype)[None, :, None, :]

        residual, h = x, None
        for i, L in enumerate(self.layers):
            if h is None:
                qkv, _ = be.norm_linear(x, L.ln1, eps, None, L.qkv)
            else:  # the previous MLP output joins the residual inside this layer's input norm
                qkv, residual = be.norm_linear(h, L.ln1, eps, residual, L.qkv)
            if merge:
                ranges = decode_attention_ranges(qkv, pos, self.inv_freq, self.k_cache[i],
                                                 self.vt_cache[i], nq, nkv, hd ** -0.5, rlen,
                                                 self.warm_set(i) if self.warm_weights and be.warms else ())
                gate_up, residual = be.attn_linear_norm_linear(ranges, L.o, residual, L.ln2, eps,
                                                               L.gate_up)
                h = be.act_linear(gate_up, L.down)
                continue
            if fused:
                attn = decode_attention(qkv, pos, self.inv_freq, self.k_cache[i], self.vt_cache[i],
                                        nq, nkv, hd ** -0.5,
                                        self.warm_set(i) if self.warm_weights and be.warms else ())
            elif prompt:
                attn = prefill_attention(qkv, pos, self.inv_freq, self.k_cache[i], self.vt_cache[i],
                                         nq, nkv, hd ** -0.5)
            else:
                q, k, v = qkv.split([nq * hd, nkv * hd, nkv * hd], dim=-1)
                q = self._rope(q.view(B, T, nq, hd), cos, sin)
                k = self._rope(k.view(B, T, nkv, hd), cos, sin)
                attn = self._attend(i, q, k, v.view(B, T, nkv, hd), pos)
            if prompt and self.fuse_prompt_act and be.fuses_prompt_act:
                act, residual = be.linear_norm_linear_act(attn, L.o, residual, L.ln2, eps, L.gate_up)
                h = be.linear(act, L.down)
            else:
                gate_up, residual = be.linear_norm_linear(attn, L.o, residual, L.ln2, eps, L.gate_up)
                h = be.act_linear(gate_up, L.down)
        if not all_logits:  # the final norm is per row: normalize the last row only
            h, residual = h[:, -1:], residual[:, -1:]
        return self._logits(h, residual)
