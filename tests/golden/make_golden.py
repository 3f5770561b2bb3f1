"""Write the small golden fixtures in this folder (tests/golden/*.npz).

Each fixture holds float64 inputs that bf16, fp16 and fp32 represent exactly
(small integers times powers of two), so every dtype sees the same values and
every product and partial sum is exact in fp32: a GPU result must then match the
expected argmax exactly, ties included. Expected outputs come from the oracle's
pure-Python loops (oracle.brute_fwd / brute_bwd), cross-checked here against the
tensor restatement before writing. The reference has no fixtures of its own.

Run:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402


def case(name, B, S, D, V, seed, bias=True, mask_kind="pad", lo=-3, hi=4, scale=0.25):
    g = torch.Generator().manual_seed(seed)
    H = torch.randint(lo, hi, (B, S, D), generator=g).double() * scale
    W = torch.randint(lo, hi, (V, D), generator=g).double() * scale
    bb = torch.randint(-2, 3, (V,), generator=g).double() * 0.125 if bias else None
    if mask_kind == "pad":
        lens = torch.randint(1, S + 1, (B,), generator=g)
        mask = (torch.arange(S)[None] < lens[:, None]).double()
    elif mask_kind == "holes":
        mask = (torch.rand(B, S, generator=g) < 0.6).double()
    elif mask_kind == "frac":
        mask = torch.randint(0, 3, (B, S), generator=g).double() * 0.5   # 0, 0.5, 1
    else:
        raise ValueError(mask_kind)
    if mask_kind != "pad" and B > 1:
        mask[0, :] = 0                                                   # an all-masked row
    G = torch.randint(0, 5, (B, V), generator=g).double() * 0.25
    M, I, reps = oracle.brute_fwd(H, W, bb, mask)
    f64 = torch.float64
    M, I, reps = torch.tensor(M, dtype=f64), torch.tensor(I), torch.tensor(reps, dtype=f64)
    tM, tI, treps = oracle.fused_fwd_ref(H, W, bb, mask)
    assert torch.equal(M, tM) and torch.equal(I, tI), name
    dH, dW, db = oracle.brute_bwd(G, reps, I, H, W, bias, mask)
    tdH, tdW, tdb = oracle.fused_bwd_ref(G, reps, I, H, W, bias, mask)
    assert torch.allclose(torch.tensor(dH, dtype=f64), tdH, rtol=1e-12, atol=1e-12), name
    assert torch.allclose(torch.tensor(dW, dtype=f64), tdW, rtol=1e-12, atol=1e-12), name
    if bias:
        assert torch.allclose(torch.tensor(db, dtype=f64), tdb, rtol=1e-12, atol=1e-12), name
    out = dict(hidden=H.numpy(), weight=W.numpy(), mask=mask.numpy(), grad=G.numpy(),
               M=M.numpy(), I=I.numpy(), reps=reps.numpy(), dH=np.array(dH), dW=np.array(dW))
    if bias:
        out["bias"] = bb.numpy()
        out["dbias"] = np.array(db)
    x = (H @ W.T + (bb if bias else 0)) * mask.unsqueeze(-1)
    ties = int((((x == M.unsqueeze(1)).sum(1) > 1) & (M > 0)).sum())
    np.savez(os.path.join(HERE, name + ".npz"), **out)
    print(f"{name}: B={B} S={S} D={D} V={V} positive={int((M > 0).sum())} tied maxima={ties}")


if __name__ == "__main__":
    case("tiny_pad_bias", 2, 6, 8, 10, seed=11)
    case("ties_pad_bias", 3, 9, 8, 24, seed=12, lo=-1, hi=2, scale=1.0)
    case("holes_nobias", 3, 7, 16, 40, seed=13, bias=False, mask_kind="holes")
    case("frac_mask_bias", 2, 5, 8, 12, seed=14, mask_kind="frac")
    case("long_s_bias", 2, 70, 8, 33, seed=15, lo=-2, hi=3, scale=0.5)
    case("two_chunks_tail", 2, 300, 8, 300, seed=16, lo=-2, hi=3, scale=0.5)
