"""GPU parity of the decode step's fused tail (``eptq_llama_lm_head_argmax``):
final RMSNorm, fp16 lm_head matvec, greedy argmax and position advance in
one launch.  The logits are within fp16 output rounding of a float32
reference (the norm restated with eptq_llama_rmsnorm's roundings, then a
float32 matmul on the CPU); the token is the first maximum of the kernel's own
fp16 logits, ties going to the smaller index as torch.argmax does; the
position advances by one; the workspace is left zeroed, so graph replays
continue the sequence."""

import numpy as np
import pytest
import torch

from eptq_amd.kernels import _lib
from eptq_amd.llama import lm_head_argmax
from oracle.matvec import rel_l2

pytestmark = pytest.mark.gpu

EPS = 1e-5


def _ref(x, delta, w, W):
    r = (x.float() + (0 if delta is None else delta.float())).half().float()
    inv = torch.rsqrt((r * r).mean(-1, keepdim=True) + EPS)
    t = (r * inv * w.float()).half().float()
    return t @ W.float().T


def _setup(B, H, V, seed, delta=True):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn((B, H), generator=gen).half()
    d = (0.5 * torch.randn((B, H), generator=gen)).half() if delta else None
    w = (1.0 + 0.05 * torch.randn(H, generator=gen)).half()
    W = (0.02 * torch.randn((V, H), generator=gen)).half()
    return x, d, w, W


def _work(B):
    return torch.zeros(_lib.load().eptq_llama_lm_head_work_bytes(B), dtype=torch.uint8, device="cuda")


@pytest.mark.parametrize("B,H,V,delta", [(1, 4096, 32000, True), (2, 4096, 1000, True), (1, 8192, 777, False),
                                         (2, 6144, 64, True), (3, 4096, 2000, True), (8, 4096, 32000, True),
                                         (5, 8192, 513, False), (8, 6144, 100, True),
                                         (8, 4096, 1537, False), (4, 4096, 5001, True)])
def test_head_matches_fp32_reference(B, H, V, delta):
    print(f"lm_head+argmax B={B} H={H} V={V} delta={delta}", flush=True)
    x, d, w, W = _setup(B, H, V, seed=B + H + V, delta=delta)
    tok = torch.full((B, 1), -1, dtype=torch.int64, device="cuda")
    pos = torch.tensor([41], dtype=torch.int64, device="cuda")
    work = _work(B)
    logits = lm_head_argmax(x.cuda(), None if d is None else d.cuda(), w.cuda(), EPS, W.cuda(), tok, pos, work)
    torch.cuda.synchronize()
    got = logits.float().cpu()
    want = _ref(x, d, w, W)
    e = rel_l2(got.numpy(), want.numpy())
    print(f"  rel_l2 {e:.2e}")
    assert e < 2e-3
    assert torch.equal(tok.cpu()[:, 0], logits.cpu().argmax(-1))   # first maximum of its own fp16 logits
    assert int(pos.item()) == 42
    assert int(work.abs().sum()) == 0


def test_head_ties_go_to_the_smaller_index():
    """Two identical lm_head rows give equal maximal logits: the smaller
    vocab index is chosen, in both batch rows."""
    print("lm_head+argmax: ties", flush=True)
    B, H, V = 2, 4096, 5000
    x, d, w, W = _setup(B, H, V, seed=9)
    W[1234] = W[4321] = (0.5 * x[0].float()).half()   # large logits for row 0
    W[77] = W[2500] = (0.5 * x[1].float()).half()
    tok = torch.zeros((B, 1), dtype=torch.int64, device="cuda")
    logits = lm_head_argmax(x.cuda(), d.cuda(), w.cuda(), EPS, W.cuda(), tok, None, _work(B))
    torch.cuda.synchronize()
    lg = logits.cpu()
    assert lg[0, 1234] == lg[0, 4321] and lg[1, 77] == lg[1, 2500]
    assert tok.cpu()[:, 0].tolist() == [int(lg[0].argmax()), int(lg[1].argmax())] == [1234, 77]


def test_head_graph_replays_advance_position():
    """Captured once, replayed several times with eager calls between: every
    replay writes the same token, advances pos by one, and leaves the
    workspace zeroed."""
    print("lm_head+argmax: graph replays", flush=True)
    B, H, V = 1, 4096, 3000
    x, d, w, W = (t.cuda() if t is not None else None for t in _setup(B, H, V, seed=3))
    tok = torch.zeros((B, 1), dtype=torch.int64, device="cuda")
    pos = torch.zeros((1,), dtype=torch.int64, device="cuda")
    work = _work(B)
    ref = lm_head_argmax(x, d, w, EPS, W, tok, pos, work).clone()
    want_tok = tok.clone()
    out = torch.empty_like(ref)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            out.copy_(lm_head_argmax(x, d, w, EPS, W, tok, pos, work))
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    p0 = int(pos.item())
    for rep in range(3):
        tok.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref) and torch.equal(tok, want_tok), rep
        assert int(pos.item()) == p0 + 2 * rep + 1, rep
        lm_head_argmax(x, d, w, EPS, W, tok, pos, work)   # eager call in between
        torch.cuda.synchronize()
        assert int(work.abs().sum()) == 0, rep


def test_decode_next_matches_decode_tokens_and_argmax():
    """The model's fused tail against the decode step's logits + torch argmax."""
    from eptq_amd.llama import LlamaConfig, build_synthetic
    print("synthetic llama: decode_next vs decode_tokens + argmax", flush=True)
    cfg = LlamaConfig(hidden=4096, ffn=1024, layers=1, heads=32, kv_heads=32, vocab=2048)
    model = build_synthetic(cfg, device="cuda", seed=21)
    for B in (1, 2, 8):
        model.alloc_cache(B, 16, "cuda")
        tok = torch.randint(0, cfg.vocab, (B, 1), device="cuda", generator=torch.Generator("cuda").manual_seed(B))
        pos = torch.tensor([3], device="cuda")
        with torch.no_grad():
            kc0 = [k.clone() for k in model.kc]
            vc0 = [v.clone() for v in model.vc]
            ref = model.decode_tokens(tok, pos)
            for i in range(cfg.layers):
                model.kc[i].copy_(kc0[i])
                model.vc[i].copy_(vc0[i])
            t2, p2 = tok.clone(), pos.clone()
            got = model.decode_next(t2, p2)
        torch.cuda.synchronize()
        assert rel_l2(got.float().cpu().numpy(), ref.float().cpu().numpy()) < 2e-3, B
        assert torch.equal(t2[:, 0].cpu(), got.cpu().argmax(-1)), B
        assert int(p2.item()) == 4


@pytest.mark.parametrize("B", [1, 8])
def test_graph_decode_with_fused_tail_crosses_the_chunk_boundary(B):
    """Greedy decode from a 250-token prompt for 12 steps (positions 250..261,
    across the attention kernel's 256-row chunk), replayed from one HIP graph
    with the fused tail, against the same steps run eagerly: same tokens at
    every step, and the fused tail (not the PyTorch fallback) ran."""
    import eptq_amd.llama as LL
    from eptq_amd.llama import GraphDecoder, LlamaConfig, build_synthetic
    print(f"synthetic llama: graph decode with fused tail, B={B}", flush=True)
    cfg = LlamaConfig(hidden=4096, ffn=1024, layers=1, heads=32, kv_heads=32, vocab=4096)
    model = build_synthetic(cfg, device="cuda", seed=31)
    dec = GraphDecoder(model, B, 272, device="cuda")
    prompt = torch.randint(0, cfg.vocab, (B, 250), device="cuda", generator=torch.Generator("cuda").manual_seed(B))
    calls = []
    real = LL.lm_head_argmax
    LL.lm_head_argmax = lambda *a, **k: (calls.append(1), real(*a, **k))[1]
    try:
        dec.prefill(prompt)
        eager = []
        for _ in range(12):
            dec.step()
            eager.append(dec.tok.clone())
        assert len(calls) == 12, "the fused tail ran at every eager step"
        assert int(dec.pos.item()) == 262
    finally:
        LL.lm_head_argmax = real
    dec.prefill(prompt)
    dec.capture()
    for i in range(12):
        dec.step()
        torch.cuda.synchronize()
        assert torch.equal(dec.tok, eager[i]), f"token {i}"
    assert int(dec.pos.item()) == 262
