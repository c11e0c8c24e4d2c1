"""Short eager programs for ``rocprofv3`` (counterpart of the reference's
``profile_kernel.py``): each case builds seeded synthetic layers on the GPU,
launches the kernel under study a few times without HIP graphs, and exits.

Counter passes (``rocprofv3 --pmc``) are run over these programs only: a few
dozen dispatches each, no graph capture.

    python -m eptq_amd.profile_cases decode --shape 4096x4096 --batch 1 --copies 8
    python -m eptq_amd.profile_cases prefill --shape 5120x5120 --tokens 2048
    python -m eptq_amd.profile_cases prefill --shape 4096x11008 --tokens 512 --work
    python -m eptq_amd.profile_cases prefill --shape 4096x4096 --tokens 2048 --bf16 --two-pass
    python -m eptq_amd.profile_cases e8 --shape 4096x4096 --batch 2048 --two-pass
    python -m eptq_amd.profile_cases e8 --shape 3072x768 --copies 8
    python -m eptq_amd.profile_cases step --layers 4
    python -m eptq_amd.profile_cases module --tokens 2048
    python -m eptq_amd.profile_cases gemm16 --shape 5120x13824 --tokens 2048
"""

from __future__ import annotations

import argparse
import sys


def _layer(torch, out, inp, seed, p, dev, qb=None, bias=False):
    from eptq_amd.synthetic import make_layer
    qd = make_layer(out, inp, seed=seed, percmask=p, qb_size=qb, bias=bias, device=dev)
    rows, cols = (qd.Q == 32767).nonzero(as_tuple=True)
    rp = torch.cat([torch.zeros(1, dtype=torch.int32, device=dev),
                    torch.bincount(rows, minlength=qd.Q.shape[0]).cumsum(0).to(torch.int32)])
    return dict(Q=qd.Q, g=qd.g, h=qd.h, O_vals=qd.O, O_col=cols.to(torch.int32), O_row_ptr=rp,
                bias=qd.bias, S_group=qd.S_group)


def main(argv=None) -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("case", choices=["decode", "prefill", "e8", "step", "module", "gemm16"])
    ap.add_argument("--shape", default="4096x4096", help="out x in")
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--tokens", type=int, default=2048)
    ap.add_argument("--copies", type=int, default=8, help="distinct layers, one launch each")
    ap.add_argument("--reps", type=int, default=2, help="passes over the copies")
    ap.add_argument("--layers", type=int, default=4, help="decoder layers (case step)")
    ap.add_argument("--qb", type=int, default=0)
    ap.add_argument("--bf16", action="store_true", help="bf16 activations (cases decode, prefill)")
    ap.add_argument("--work", action="store_true",
                    help="through the multi-layer entry point with a decode workspace (split K; cases decode, prefill)")
    ap.add_argument("--two-pass", action="store_true",
                    help="the module's route (two passes from its token thresholds; cases prefill, e8)")
    args = ap.parse_args(argv)

    import torch
    from eptq_amd.kernels import linear_forward, linear_forward_multi, decode_workspace
    from eptq_amd.quantizers import E8D4Quantizer, E8LatticeQuantizer
    from eptq_amd.synthetic import make_x

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    out, inp = (int(v) for v in args.shape.split("x"))
    qb = args.qb or None
    if args.case in ("decode", "prefill"):
        codes = E8D4Quantizer(radius=1.75).flat_table().half().to(dev)
        T = args.batch if args.case == "decode" else args.tokens
        layers = [_layer(torch, out, inp, 7000 + c, 0.001, dev, qb=qb) for c in range(args.copies)]
        x = make_x(T, inp, seed=1, device=dev)
        if args.bf16:
            x = x.bfloat16()
        work = decode_workspace(dev) if args.work else None
        torch.cuda.synchronize()
        for _ in range(args.reps):
            for L in layers:
                if work is not None:
                    linear_forward_multi([L], codes, x, work=work)
                else:
                    linear_forward("e8_d4", L["Q"], codes, L["g"], L["h"], x, L["O_vals"], L["O_col"],
                                   L["O_row_ptr"], None, L["S_group"], two_pass=args.two_pass)
    elif args.case == "e8":
        codes = E8LatticeQuantizer(radius=1.6).flat_table().half().to(dev)
        layers = [_layer(torch, out, inp, 7100 + c, 0.002, dev, bias=True) for c in range(args.copies)]
        x = make_x(args.batch, inp, seed=2, device=dev)
        torch.cuda.synchronize()
        for _ in range(args.reps):
            for L in layers:
                linear_forward("e8_lattice", L["Q"], codes, L["g"], L["h"], x, L["O_vals"], L["O_col"],
                               L["O_row_ptr"], L["bias"], None, two_pass=args.two_pass)
    elif args.case == "gemm16":
        # The two-pass prefill's second pass alone (eptq_f16_gemm) on a seeded
        # fp16 W (out x in) and x (--tokens x in), --reps launches.
        from eptq_amd.kernels import f16_gemm
        gen = torch.Generator(device=dev).manual_seed(5)
        W = (torch.randn((out, inp), generator=gen, device=dev) * 0.05).half()
        x = torch.randn((args.tokens, inp), generator=gen, device=dev).half()
        torch.cuda.synchronize()
        for _ in range(args.reps):
            f16_gemm(W, x)
    elif args.case == "module":
        # One Llama-2-13B decoder layer's Linears through the drop-in modules
        # (EPTQMultiLinear q|k|v and gate|up, EPTQLinear o and down) at
        # --tokens rows: the kernels the module forward runs.
        from eptq_amd.kernels.linear import EPTQLinear, EPTQMultiLinear
        from eptq_amd.synthetic import make_layer
        q = E8D4Quantizer(radius=1.75)

        def mod(o, i, k):
            return EPTQLinear.from_quantized_data(make_layer(o, i, seed=9000 + k, percmask=0.002, device=dev),
                                                  q, "e8_d4").to(dev)
        d = 5120
        mods = [EPTQMultiLinear([mod(d, d, k) for k in range(3)]), mod(d, d, 3),
                EPTQMultiLinear([mod(13824, d, 4), mod(13824, d, 5)]), mod(d, 13824, 6)]
        xs = {n: make_x(args.tokens, n, seed=n, device=dev) for n in (d, 13824)}
        torch.cuda.synchronize()
        with torch.no_grad():
            for _ in range(args.reps):
                for m in mods:
                    m(xs[m.in_features])
    else:
        # One decode step's Linear units of args.layers Llama-2-7B layers:
        # q|k|v and gate|up as multi-layer launches, o and down alone.
        codes = E8D4Quantizer(radius=1.75).flat_table().half().to(dev)
        work = decode_workspace(dev)
        units = []
        for li in range(args.layers):
            mk = lambda o, i, k: _layer(torch, o, i, 8000 + 10 * li + k, 0.001, dev)
            units.append([mk(4096, 4096, k) for k in range(3)])
            units.append([mk(4096, 4096, 3)])
            units.append([mk(11008, 4096, 4), mk(11008, 4096, 5)])
            units.append([mk(4096, 11008, 6)])
        xs = {n: make_x(args.batch, n, seed=n, device=dev) for n in (4096, 11008)}
        torch.cuda.synchronize()
        for _ in range(args.reps):
            for u in units:
                linear_forward_multi(u, codes, xs[int(u[0]["Q"].shape[1])], work=work)
    torch.cuda.synchronize()
    print(f"profile case {args.case} done", flush=True)


if __name__ == "__main__":
    main(sys.argv[1:])
