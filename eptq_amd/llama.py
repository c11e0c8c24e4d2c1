"""Self-contained Llama decoder whose Linears are ``EPTQLinear`` (synthetic weights).

Counterpart of the reference's decode benchmark driver (``bench_decode.py:44-71``:
prefill untimed, then a timed token-by-token loop over a static KV cache),
without HuggingFace model loading: the model is built from its config with
every decoder Linear (q/k/v/o, gate/up/down) a synthetic E8-D4
``QuantizedLayerData`` and the embedding, norms and ``lm_head`` random fp16
(the reference keeps ``lm_head`` unquantized, ``quantize.py:86-90``).

Decode step (one token per sequence), 5 launches per layer: q|k|v with the
RMSNorm formed inside the launch (one multi-layer decode launch) -> rotary +
cache write + attention (one kernel) -> o -> gate|up with the RMSNorm inside
and silu(gate)·up at its output -> down, the residual adds inside the o and
down launches (B <= 2: inside the q|k|v and gate|up launches).  Shapes are
static (preallocated cache, position in a device tensor), so the step is
captured once in a HIP graph and replayed.
Prefill (many tokens) runs the same Linears (MFMA GEMM) and PyTorch attention.
Greedy decoding.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from .kernels import _lib, decode_workspace
from .kernels.linear import EPTQLinear, EPTQMultiLinear
from .quantizers import E8D4Quantizer
from .synthetic import make_layer


@dataclass
class LlamaConfig:
    hidden: int = 4096
    ffn: int = 11008
    layers: int = 32
    heads: int = 32
    kv_heads: int = 32
    vocab: int = 32000
    rope_theta: float = 10000.0
    eps: float = 1e-5

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads


LLAMA2_7B = LlamaConfig()


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def rmsnorm_(x: torch.Tensor, delta: Optional[torch.Tensor], w: torch.Tensor, eps: float) -> torch.Tensor:
    """x += delta (in place, if given); returns w ⊙ x / rms(x) (HIP kernel)."""
    B, H = x.shape
    y = torch.empty_like(x)
    rc = _lib.load().eptq_llama_rmsnorm(x.data_ptr(), None if delta is None else delta.data_ptr(),
                                        w.data_ptr(), y.data_ptr(), B, H, eps, _stream(x))
    _lib.check(rc, "eptq_llama_rmsnorm")
    return y


def silu_mul(gu: torch.Tensor) -> torch.Tensor:
    B, F2 = gu.shape
    a = torch.empty((B, F2 // 2), dtype=gu.dtype, device=gu.device)
    _lib.check(_lib.load().eptq_llama_silu_mul(gu.data_ptr(), a.data_ptr(), B, F2 // 2, _stream(gu)),
               "eptq_llama_silu_mul")
    return a


def _layer_array(lins):
    """``eptq_layer`` array for E8-D4 ``EPTQLinear`` parts, outputs side by side."""
    arr = (_lib.EptqLayer * len(lins))()
    off = 0
    for k, l in enumerate(lins):
        def p(t):
            return None if t is None or t.numel() == 0 else t.data_ptr()
        n_groups = 0 if l.S_group is None else int(l.S_group.shape[0])
        arr[k] = _lib.EptqLayer(p(l.Q), p(l.g), p(l.h), p(l.O_vals), p(l.O_col), p(l.O_row_ptr), p(l.bias),
                                p(l.S_group), n_groups, int(l.Q.shape[0]), off)
        off += l.out_features
    return arr, off


def _parts(mod):
    return list(mod.parts) if isinstance(mod, EPTQMultiLinear) else [mod]


def _array_key(lins):
    """Every pointer, dtype and size the layer array carries: a buffer that is
    reassigned, moved or converted changes the key."""
    key = []
    for l in lins:
        for t in (l.Q, l.g, l.h, l.O_vals, l.O_col, l.O_row_ptr, l.bias, l.S_group, l._codebook):
            key.append(None if t is None else (t.data_ptr(), t.dtype, tuple(t.shape), str(t.device)))
    return tuple(key)


def _cached_array(mod):
    key = _array_key(_parts(mod))
    cached = getattr(mod, "_eptq_array", None)
    if cached is None or cached[0] != key:
        cached = (key, *_layer_array(_parts(mod)))
        mod._eptq_array = cached
    return cached[1], cached[2]


def norm_linear(mod, resid, delta, w, eps, resid_out):
    """mod(RMSNorm(resid + delta)) with the norm fused into the decode launch;
    resid + delta is written to resid_out (if given).  Raises EptqError
    (code EPTQ_EUNSUPPORTED) when the kernel cannot take the shape."""
    arr, width = _cached_array(mod)
    B, N = resid.shape
    y = torch.empty((B, width), dtype=resid.dtype, device=resid.device)
    rc = _lib.load().eptq_llama_norm_linear(
        len(arr), arr, _parts(mod)[0]._codebook.data_ptr(), resid.data_ptr(),
        None if delta is None else delta.data_ptr(), w.data_ptr(), eps,
        None if resid_out is None else resid_out.data_ptr(), N, B, y.data_ptr(), width, _stream(resid))
    _lib.check(rc, "eptq_llama_norm_linear")
    return y


def norm_swiglu(mod, resid, delta, w, eps, resid_out):
    """silu(gate(t)) * up(t) for t = RMSNorm(resid + delta), ``mod`` the fused
    gate|up module, in one decode launch; resid + delta is written to
    resid_out (if given).  Raises EptqError (code EPTQ_EUNSUPPORTED) when the
    kernel cannot take the shape or batch."""
    arr, width = _cached_array(mod)
    B, N = resid.shape
    out = torch.empty((B, width // 2), dtype=resid.dtype, device=resid.device)
    rc = _lib.load().eptq_llama_norm_swiglu(
        arr, _parts(mod)[0]._codebook.data_ptr(), resid.data_ptr(), None if delta is None else delta.data_ptr(),
        w.data_ptr(), eps, None if resid_out is None else resid_out.data_ptr(), N, B, out.data_ptr(), _stream(resid))
    _lib.check(rc, "eptq_llama_norm_swiglu")
    return out


def lm_head_argmax(x, delta, w, eps, W, tok, pos, work):
    """logits (B, V) = RMSNorm(x + delta) · Wᵀ, tok[:, 0] <- argmax, pos += 1,
    in one launch.  Raises EptqError (code EPTQ_EUNSUPPORTED) for B > 8 or an
    unsupported hidden size."""
    B, H = x.shape
    V = W.shape[0]
    logits = torch.empty((B, V), dtype=x.dtype, device=x.device)
    rc = _lib.load().eptq_llama_lm_head_argmax(
        x.data_ptr(), None if delta is None else delta.data_ptr(), w.data_ptr(), eps, W.data_ptr(), V, H, B,
        logits.data_ptr(), tok.data_ptr(), None if pos is None else pos.data_ptr(), work.data_ptr(), _stream(x))
    _lib.check(rc, "eptq_llama_lm_head_argmax")
    return logits


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim, dtype=torch.float16), requires_grad=False)
        self.eps = eps

    def forward(self, x):
        xf = x.float()
        xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        return (xf * self.weight.float()).to(x.dtype)


def _rope(x, cos, sin):
    # x: (B, H, T, D); rotate halves as in the HF Llama implementation
    d = x.shape[-1] // 2
    x1, x2 = x[..., :d], x[..., d:]
    rot = torch.cat((-x2, x1), dim=-1)
    return (x.float() * cos + rot.float() * sin).to(x.dtype)


class DecoderLayer(nn.Module):
    def __init__(self, cfg: LlamaConfig, lin: dict):
        super().__init__()
        self.cfg = cfg
        self.input_layernorm = RMSNorm(cfg.hidden, cfg.eps)
        self.post_attention_layernorm = RMSNorm(cfg.hidden, cfg.eps)
        self.qkv_proj = EPTQMultiLinear([lin["q_proj"], lin["k_proj"], lin["v_proj"]])
        self.o_proj = lin["o_proj"]
        self.gate_up_proj = EPTQMultiLinear([lin["gate_proj"], lin["up_proj"]])
        self.down_proj = lin["down_proj"]

    def forward(self, x, cos, sin, kc, vc, pos, mask):
        """Prefill (T tokens): x (B, T, hidden); caches (B, Hkv, L, D); pos (T,)
        positions; mask (T, L) additive.  PyTorch attention."""
        cfg = self.cfg
        B, T, _ = x.shape
        H, Hk, D = cfg.heads, cfg.kv_heads, cfg.head_dim
        h = self.input_layernorm(x)
        qkv = self.qkv_proj(h)
        q, k, v = qkv.split([H * D, Hk * D, Hk * D], dim=-1)
        q = _rope(q.reshape(B, T, H, D).transpose(1, 2), cos, sin).contiguous()
        k = _rope(k.reshape(B, T, Hk, D).transpose(1, 2), cos, sin)
        v = v.reshape(B, T, Hk, D).transpose(1, 2)
        kc.index_copy_(2, pos, k)
        vc.index_copy_(2, pos, v)
        kk, vv = kc, vc
        if Hk != H:
            kk = kk.repeat_interleave(H // Hk, dim=1)
            vv = vv.repeat_interleave(H // Hk, dim=1)
        s = torch.matmul(q.float(), kk.float().transpose(-1, -2).contiguous()) * (1.0 / math.sqrt(D)) + mask
        p = torch.softmax(s, dim=-1)
        o = torch.matmul(p, vv.float()).to(x.dtype)
        o = o.transpose(1, 2).reshape(B, T, H * D)
        x = x + self.o_proj(o)
        h = self.post_attention_layernorm(x)
        gu = self.gate_up_proj(h).float()
        a = F.silu(gu[..., :cfg.ffn]) * gu[..., cfg.ffn:]
        return x + self.down_proj(a.to(x.dtype))


class QuantLlama(nn.Module):
    """Llama with EPTQ-quantized decoder Linears and a static KV cache."""

    def __init__(self, cfg: LlamaConfig, layers: List[DecoderLayer], embed, norm, lm_head):
        super().__init__()
        self.cfg = cfg
        self.layers = nn.ModuleList(layers)
        self.embed_tokens = embed
        self.norm = norm
        self.lm_head = lm_head
        self.kc: Optional[list] = None
        self.split_attention = False
        # Decode step: the residual add + RMSNorm inside the q|k|v and gate|up
        # launches (B <= 2: the vector kernel; 3..8: the matrix-core kernel,
        # with the adds in the o and down launches) or as launches of their own.
        self.fused_ops = True

    def alloc_cache(self, batch: int, max_len: int, device):
        cfg = self.cfg
        shape = (batch, cfg.kv_heads, max_len, cfg.head_dim)
        self.kc = [torch.zeros(shape, dtype=torch.float16, device=device) for _ in self.layers]
        self.vc = [torch.zeros(shape, dtype=torch.float16, device=device) for _ in self.layers]
        self.max_len = max_len
        inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, cfg.head_dim, 2, device=device).float() / cfg.head_dim))
        t = torch.arange(max_len, device=device).float()
        f = torch.outer(t, inv)
        emb = torch.cat((f, f), dim=-1)
        self.cos_tab, self.sin_tab = emb.cos().contiguous(), emb.sin().contiguous()
        # Split-position attention (a workspace of partials and zeroed
        # counters) only on request: at these context lengths one workgroup
        # per (head, sequence) measured faster than splitting and combining.
        self.attn_work = None
        if self.split_attention:
            nbytes = _lib.load().eptq_llama_attn_work_bytes(batch, cfg.heads)
            self.attn_work = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        # Split-K workspace of the decode Linears (batches of 3..16, and the
        # 16-token slices of short prefills through the modules): the model's
        # launches run one after another on one stream.
        self.lin_work = decode_workspace(device)
        for m in self.modules():
            if isinstance(m, (EPTQLinear, EPTQMultiLinear)):
                m._work = self.lin_work
        # Workspace of the fused final norm + lm_head + argmax (B <= 8).
        self.head_work = None
        if batch <= 8:
            nbytes = _lib.load().eptq_llama_lm_head_work_bytes(batch)
            self.head_work = torch.zeros(nbytes, dtype=torch.uint8, device=device)

    def forward_tokens(self, ids, pos):
        """ids: (B, T) int64, pos: (T,) int64 positions -> logits (B, T, vocab)."""
        x = self.embed_tokens(ids)
        T = ids.shape[1]
        cos = self.cos_tab.index_select(0, pos)[None, None]
        sin = self.sin_tab.index_select(0, pos)[None, None]
        L = self.max_len
        allowed = torch.arange(L, device=ids.device)[None, :] <= pos[:, None]
        mask = torch.zeros((T, L), dtype=torch.float32, device=ids.device).masked_fill(~allowed, float("-inf"))
        for i, layer in enumerate(self.layers):
            x = layer(x, cos, sin, self.kc[i], self.vc[i], pos, mask)
        x = self.norm(x)
        return self.lm_head(x)

    def _lin(self, mod, x):
        """mod(x) for a decode step: the E8-D4 parts of ``mod`` in one launch
        of the multi-layer entry point, with the step's split-K workspace."""
        arr, width = _cached_array(mod)
        B, N = x.shape
        y = torch.empty((B, width), dtype=x.dtype, device=x.device)
        work = getattr(self, "lin_work", None)
        rc = _lib.load().eptq_e8d4_forward_multi(
            len(arr), arr, _parts(mod)[0]._codebook.data_ptr(), _lib.EPTQ_F16, x.data_ptr(), _lib.EPTQ_F16,
            N, B, y.data_ptr(), width, None if work is None else work.data_ptr(),
            0 if work is None else work.numel(), _stream(x))
        _lib.check(rc, "eptq_e8d4_forward_multi")
        return y

    def _llin(self, mod, x, norm_w=None, resid=None):
        """mod(t) on the matrix-core decode kernel (``eptq_llama_linear``),
        t = x or RMSNorm(x) with weight norm_w; with resid the result is added
        to resid in place and resid returned."""
        arr, width = _cached_array(mod)
        B, N = x.shape
        y = resid if resid is not None else torch.empty((B, width), dtype=x.dtype, device=x.device)
        work = getattr(self, "lin_work", None)
        rc = _lib.load().eptq_llama_linear(
            len(arr), arr, _parts(mod)[0]._codebook.data_ptr(), x.data_ptr(), N, B,
            None if norm_w is None else norm_w.data_ptr(), self.cfg.eps,
            None if resid is None else resid.data_ptr(), y.data_ptr(), width,
            None if work is None else work.data_ptr(), 0 if work is None else work.numel(), _stream(x))
        _lib.check(rc, "eptq_llama_linear")
        return y

    def _llin_swiglu(self, mod, x, norm_w):
        """silu(gate(t)) * up(t), t = RMSNorm(x) with weight norm_w, on the
        matrix-core decode kernel with the product formed in the same launch
        (``eptq_llama_linear_swiglu``, which needs the step's workspace);
        without a workspace the gate|up launch and the SiLU kernel."""
        work = getattr(self, "lin_work", None)
        if work is None:
            return silu_mul(self._llin(mod, x, norm_w=norm_w))
        arr, width = _cached_array(mod)
        B, N = x.shape
        gu = torch.empty((B, width), dtype=x.dtype, device=x.device)
        act = torch.empty((B, width // 2), dtype=x.dtype, device=x.device)
        rc = _lib.load().eptq_llama_linear_swiglu(
            arr, _parts(mod)[0]._codebook.data_ptr(), x.data_ptr(), N, B,
            None if norm_w is None else norm_w.data_ptr(), self.cfg.eps, gu.data_ptr(), act.data_ptr(),
            work.data_ptr(), work.numel(), _stream(x))
        _lib.check(rc, "eptq_llama_linear_swiglu")
        return act

    def _norm_into(self, mod, x, delta, w):
        """mod(RMSNorm(x + delta)) and the residual x + delta (a new tensor when
        fused; x itself, updated in place, on the separate-launch path)."""
        if self.fused_ops:
            r = torch.empty_like(x) if delta is not None else None
            try:
                return norm_linear(mod, x, delta, w, self.cfg.eps, r), (x if r is None else r)
            except _lib.EptqError as e:
                if e.code != _lib.EPTQ_EUNSUPPORTED:
                    raise
        return self._lin(mod, rmsnorm_(x, delta, w, self.cfg.eps)), x

    def _norm_swiglu(self, mod, x, delta, w):
        """silu(gate) * up of RMSNorm(x + delta) and the residual, in one launch
        where the kernel takes it (fused ops, B <= 2), else as the fused-norm
        gate|up launch followed by the SiLU kernel."""
        if self.fused_ops and x.shape[0] <= 2:
            r = torch.empty_like(x) if delta is not None else None
            try:
                return norm_swiglu(mod, x, delta, w, self.cfg.eps, r), (x if r is None else r)
            except _lib.EptqError as e:
                if e.code != _lib.EPTQ_EUNSUPPORTED:
                    raise
        gu, x = self._norm_into(mod, x, delta, w)
        return silu_mul(gu), x

    def decode_tokens(self, tok, pos):
        """One token per sequence: tok (B, 1) int64, pos (1,) int64 on the device
        -> logits (B, vocab).  HIP kernels for everything but the embedding,
        lm_head and argmax; with ``fused_ops`` the norms run inside the Linear
        launches (norm(+residual) -> q|k|v, attention, o, norm(+residual) ->
        gate|up -> silu·up, down; for B <= 2 the SwiGLU product is formed in
        the gate|up launch itself, whose workgroups compute the same rows of
        both layers, otherwise it is a launch of its own)."""
        x, delta = self._decode_layers(tok, pos)
        h = rmsnorm_(x, delta, self.norm.weight, self.cfg.eps)
        return self.lm_head(h)

    def _matrix_core_step(self, B):
        """Whether a decode step of B rows runs its Linears on the matrix-core
        kernel with the norms, residual adds and SwiGLU product folded in (5
        launches per layer): 3 <= B <= 8, fp16, hidden a multiple of 64."""
        return (self.fused_ops and 3 <= B <= 8 and self.cfg.hidden % 64 == 0
                and self.embed_tokens.weight.dtype == torch.float16)

    def _decode_layers(self, tok, pos):
        """The decoder layers of one decode step: the residual stream x and the
        last layer's output delta (their sum is the final norm's input; delta
        is None when the last add is already in x)."""
        cfg = self.cfg
        H, Hk, D = cfg.heads, cfg.kv_heads, cfg.head_dim
        x = self.embed_tokens(tok[:, 0])                    # (B, hidden), the residual stream
        B = x.shape[0]
        lib = _lib.load()
        delta = None
        mc = self._matrix_core_step(B)
        for i, layer in enumerate(self.layers):
            ln1, ln2 = layer.input_layernorm.weight, layer.post_attention_layernorm.weight
            if mc:
                qkv = self._llin(layer.qkv_proj, x, norm_w=ln1)
            else:
                qkv, x = self._norm_into(layer.qkv_proj, x, delta, ln1)
            att = torch.empty((B, H * D), dtype=x.dtype, device=x.device)
            rc = lib.eptq_llama_rope_attn(qkv.data_ptr(), pos.data_ptr(), self.cos_tab.data_ptr(),
                                          self.sin_tab.data_ptr(), self.kc[i].data_ptr(), self.vc[i].data_ptr(),
                                          att.data_ptr(), B, H, Hk, D, self.max_len,
                                          None if self.attn_work is None else self.attn_work.data_ptr(),
                                          _stream(x))
            _lib.check(rc, "eptq_llama_rope_attn")
            if mc:
                self._llin(layer.o_proj, att, resid=x)                 # x += o(att)
                act = self._llin_swiglu(layer.gate_up_proj, x, ln2)
                self._llin(layer.down_proj, act, resid=x)              # x += down(act)
                continue
            o = self._lin(layer.o_proj, att)
            act, x = self._norm_swiglu(layer.gate_up_proj, x, o, ln2)
            delta = self._lin(layer.down_proj, act)
        return x, delta

    def decode_next(self, tok, pos):
        """One greedy step in place: logits (B, vocab) for tok at pos, then
        tok <- argmax(logits) and pos += 1.  With ``fused_ops`` and B <= 8
        the final norm, lm_head, argmax and position advance are one launch
        (``eptq_llama_lm_head_argmax``); otherwise PyTorch's lm_head and
        argmax follow the decode step."""
        x, delta = self._decode_layers(tok, pos)
        W = self.lm_head.weight
        if self.fused_ops and self.head_work is not None and W.dtype == torch.float16 and W.is_contiguous():
            try:
                return lm_head_argmax(x, delta, self.norm.weight, self.cfg.eps, W, tok, pos, self.head_work)
            except _lib.EptqError as e:
                if e.code != _lib.EPTQ_EUNSUPPORTED:
                    raise
        logits = self.lm_head(rmsnorm_(x, delta, self.norm.weight, self.cfg.eps))
        tok.copy_(logits.argmax(-1, keepdim=True))
        pos.add_(1)
        return logits


def build_synthetic(cfg: LlamaConfig = LLAMA2_7B, device="cuda", seed: int = 4000,
                    percmask: float = 0.002, radius: float = 1.75) -> QuantLlama:
    """Random-init Llama whose decoder Linears are synthetic E8-D4 layers."""
    quant = E8D4Quantizer(device=str(device), radius=radius)
    shapes = {"q_proj": (cfg.hidden, cfg.hidden),
              "k_proj": (cfg.kv_heads * cfg.head_dim, cfg.hidden),
              "v_proj": (cfg.kv_heads * cfg.head_dim, cfg.hidden),
              "o_proj": (cfg.hidden, cfg.hidden),
              "gate_proj": (cfg.ffn, cfg.hidden),
              "up_proj": (cfg.ffn, cfg.hidden),
              "down_proj": (cfg.hidden, cfg.ffn)}
    gen = torch.Generator(device=device).manual_seed(seed)
    layers = []
    for li in range(cfg.layers):
        lin = {}
        for idx, (name, (out, inp)) in enumerate(shapes.items()):
            qd = make_layer(out, inp, seed=seed + 10 * li + idx, percmask=percmask, device=device)
            lin[name] = EPTQLinear.from_quantized_data(qd, quant, "e8_d4")
        layer = DecoderLayer(cfg, lin)
        with torch.no_grad():
            layer.input_layernorm.weight.copy_(1.0 + 0.05 * torch.randn(cfg.hidden, generator=gen, device=device))
            layer.post_attention_layernorm.weight.copy_(1.0 + 0.05 * torch.randn(cfg.hidden, generator=gen, device=device))
        layers.append(layer.to(device))
    embed = nn.Embedding(cfg.vocab, cfg.hidden).to(device=device, dtype=torch.float16)
    lm_head = nn.Linear(cfg.hidden, cfg.vocab, bias=False).to(device=device, dtype=torch.float16)
    norm = RMSNorm(cfg.hidden, cfg.eps).to(device)
    with torch.no_grad():
        embed.weight.copy_(torch.randn(cfg.vocab, cfg.hidden, generator=gen, device=device) * 0.02)
        lm_head.weight.copy_(torch.randn(cfg.vocab, cfg.hidden, generator=gen, device=device) * 0.02)
    embed.weight.requires_grad_(False)
    lm_head.weight.requires_grad_(False)
    return QuantLlama(cfg, layers, embed, norm, lm_head).eval()


class GraphDecoder:
    """Greedy decode with the per-token step captured in a HIP graph.

    ``fused=True`` runs the step on the fused decode kernels
    (``QuantLlama.decode_tokens``); ``fused=False`` on the PyTorch-attention
    path used for prefill (``forward_tokens``), kept as a cross-check."""

    def __init__(self, model: QuantLlama, batch: int, max_len: int, device="cuda", fused: bool = True):
        self.model = model
        self.batch = batch
        self.fused = fused
        self.device = torch.device(device)
        model.alloc_cache(batch, max_len, self.device)
        # The buffers this decoder's launches address (held, so a captured
        # graph never addresses freed memory).  A later GraphDecoder on the
        # same model replaces them in the model; this one then refuses to run.
        self._bufs = self._model_bufs()
        self.tok = torch.zeros((batch, 1), dtype=torch.long, device=self.device)
        self.pos = torch.zeros((1,), dtype=torch.long, device=self.device)
        self.graph = None

    def _model_bufs(self):
        m = self.model
        return (m.kc, m.vc, m.cos_tab, m.sin_tab, m.attn_work, m.lin_work, m.head_work)

    def _check_owner(self):
        if any(a is not b for a, b in zip(self._model_bufs(), self._bufs)):
            raise RuntimeError("the model's caches and workspaces now belong to a newer GraphDecoder; "
                               "this decoder (and its captured graph) can no longer run")

    @torch.no_grad()
    def prefill(self, prompt: torch.Tensor) -> torch.Tensor:
        self._check_owner()
        T = prompt.shape[1]
        pos = torch.arange(T, device=self.device)
        logits = self.model.forward_tokens(prompt, pos)
        nxt = logits[:, -1].argmax(-1, keepdim=True)
        self.tok.copy_(nxt)
        self.pos.fill_(T)
        return nxt

    @torch.no_grad()
    def _step(self):
        if self.fused:
            self.model.decode_next(self.tok, self.pos)
        else:
            logits = self.model.forward_tokens(self.tok, self.pos)[:, -1]
            self.tok.copy_(logits.argmax(-1, keepdim=True))
            self.pos.add_(1)

    @torch.no_grad()
    def capture(self):
        self._check_owner()
        # Warm up on a side stream (allocator and kernels), then capture.
        saved_tok, saved_pos = self.tok.clone(), self.pos.clone()
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            self._step()
        torch.cuda.current_stream(self.device).wait_stream(side)
        self.tok.copy_(saved_tok)
        self.pos.copy_(saved_pos)
        torch.cuda.synchronize(self.device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._step()
        self.tok.copy_(saved_tok)
        self.pos.copy_(saved_pos)
        torch.cuda.synchronize(self.device)

    def step(self):
        self._check_owner()
        if self.graph is None:
            self._step()
        else:
            self.graph.replay()
