"""GPU parity: the HIP kernels (through the C ABI via the torch ops) against the CPU
oracle on identical, seeded, already-rounded inputs. Every test prints its case
before touching the GPU."""
import glob
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
import sparton
from sparton_amd import _lib
from sparton_amd.workloads import WORKLOADS, make_inputs
from _parity import (BWD_TOL, F64, FWD_TOL, check_bwd_isolated, check_dw_identity_gpu,
                     check_fwd, check_fwd_full_gpu, say)

pytestmark = pytest.mark.gpu

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))
DTYPES = {"fp32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16}


def run_fwd_bwd(H, W, b, m, G, device):
    """Training path: fwd_train, then the backward from its unrounded fp32 reps.
    Also checks that the reference-signature forward returns the same reps/idx."""
    Hd, Wd, md, Gd = H.to(device), W.to(device), m.to(device), G.to(device)
    bd = None if b is None else b.to(device)
    reps, idx, reps32 = torch.ops.sparton.fused_sparton_fwd_train(Hd, Wd, bd, md)
    r2, i2 = torch.ops.sparton.fused_sparton_fwd(Hd, Wd, bd, md)
    assert torch.equal(reps, r2) and torch.equal(idx, i2)
    assert torch.equal(reps32.to(reps.dtype), reps)
    dH, dW, db = torch.ops.sparton.fused_sparton_bwd(Gd, reps32, idx, Hd, Wd, bd, md)
    torch.cuda.synchronize()
    return reps, idx, reps32, dH, dW, db


@pytest.mark.parametrize("dt", list(DTYPES))
@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p)[:-4] for p in GOLDEN])
def test_golden_fixture_exact_argmax(path, dt, device):
    """Inputs are exact in every dtype and all partial sums are exact in fp32, so the
    argmax must match exactly, ties included (lowest s)."""
    z = np.load(path)
    t = {k: torch.from_numpy(z[k]) for k in z.files}
    dtype = DTYPES[dt]
    H, W = t["hidden"].to(dtype), t["weight"].to(dtype)
    b = t["bias"].to(dtype) if "bias" in t else None
    m, G = t["mask"].to(torch.float32), t["grad"].to(dtype)
    say(f"golden {os.path.basename(path)} {dt} B,S,D,V={tuple(H.shape)}+{W.shape[0]}")
    reps, idx, reps32, dH, dW, db = run_fwd_bwd(H, W, b, m, G, device)
    assert torch.equal(idx.cpu().long(), t["I"])
    torch.testing.assert_close(reps.cpu().to(F64), t["reps"], **FWD_TOL)
    torch.testing.assert_close(reps32.cpu().to(F64), t["reps"], rtol=1e-6, atol=1e-6)
    # training path (fp32 reps): matches the fp64 fixture to fp32 accuracy
    torch.testing.assert_close(dH.cpu().to(F64), t["dH"], **BWD_TOL)
    torch.testing.assert_close(dW.cpu().to(F64), t["dW"], **BWD_TOL)
    if b is not None:
        torch.testing.assert_close(db.cpu().to(F64), t["dbias"], **BWD_TOL)
    # reference-signature path (rounded reps, sparton_kernel.py:531): the oracle at those reps
    Hd, Wd, md, Gd = H.to(device), W.to(device), m.to(device), G.to(device)
    bd = None if b is None else b.to(device)
    dH2, dW2, db2 = torch.ops.sparton.fused_sparton_bwd(Gd, reps, idx, Hd, Wd, bd, md)
    check_bwd_isolated(H, W, b, m, G, reps, idx, dH2, dW2, db2)


CASES = [
    # dtype, B, S, D, V, bias, mask kind
    ("bf16", 3, 77, 64, 1000, True, "int64"),
    ("fp16", 2, 300, 128, 777, False, "bool"),
    ("fp32", 2, 40, 96, 513, True, "frac"),
    ("bf16", 1, 600, 256, 300, True, "int32"),
    ("bf16", 4, 1, 32, 100, True, "int64"),
    ("bf16", 2, 256, 768, 4099, True, "holes"),
    ("fp16", 3, 33, 16, 70, True, "f16"),
    ("fp32", 1, 5, 4, 1, False, "int64"),
    ("bf16", 2, 50, 72, 300, True, "int64"),    # K tail: 144-byte rows (2 slabs + tail)
    ("fp32", 2, 20, 40, 260, False, "holes"),   # K tail: 160-byte rows
    ("fp16", 3, 130, 24, 520, True, "int64"),   # rows shorter than one slab, 3 vocab tiles
    ("bf16", 3, 900, 64, 2100, True, "gaps"),   # fully masked middle chunk, masked row
    ("bf16", 37, 40, 64, 700, True, "int64"),   # many short rows: several rows per row tile
    ("fp32", 130, 3, 16, 70, True, "int64"),    # B > 128: staged dW, 64 ids per workgroup
    ("fp32", 300, 4, 40, 333, True, "holes"),   # B > 256: staged dW, 32 ids per workgroup
    ("bf16", 250, 6, 264, 500, False, "frac"),  # staged dW, 64 ids, two passes with a tail
    ("fp16", 1024, 2, 8, 50, True, "bool"),     # B = 1024: staged dW, 16 ids per workgroup
    ("fp32", 700, 3, 16, 90, True, "int64"),    # fp32 B > 512: the unstaged dW path
    ("bf16", 100, 24, 64, 900, True, "frac"),   # 64 < B <= 128: staged dW, two batch passes
    ("bf16", 8, 3000, 64, 700, True, "gaps"),   # B*S > 16384: plan with the mask in global memory
    ("fp16", 1100, 8, 16, 200, True, "int64"),  # more groups than plan threads
    ("bf16", 600, 500, 16, 300, True, "holes"),  # > 16384 groups: the three-kernel plan
    ("fp16", 6, 70, 32, 333, False, "bf16"),    # bf16 mask
]

# Cases run again with several vocab tiles per workgroup (the unit stream then crosses
# vocab tiles and chunks inside one workgroup, including a partial last group).
# (case, grid): the persistent forward kernel run with `grid` workgroups, so each
# walks many units. nk = K slabs per unit; nk >= 4 fetches the next unit's metadata
# inside the K loop, nk < 4 hands over synchronously.
PERSISTENT_CASES = [
    (("bf16", 3, 900, 64, 2100, True, "gaps"), 1),      # nk 2, one workgroup for all units
    (("fp32", 2, 40, 96, 1300, True, "frac"), 2),       # nk 3
    (("fp16", 2, 300, 24, 1800, False, "bool"), 4),     # nk 2 (K tail)
    (("bf16", 2, 256, 768, 4099, True, "holes"), 3),    # nk 12
    (("fp16", 37, 40, 64, 700, True, "int64"), 9),
    (("fp32", 3, 70, 132, 900, True, "frac"), 5),       # nk 5 (K tail), fractional mask
    (("fp16", 5, 100, 200, 1500, False, "gaps"), 7),    # nk 4 (K tail)
    (("bf16", 37, 40, 256, 700, True, "int64"), 13),    # nk 4, tiles spanning batch rows
    (("bf16", 6, 200, 296, 3000, True, "gaps"), 5),     # nk 5 (K tail), metadata prefetched
    (("fp16", 4, 128, 1024, 2000, False, "frac"), 6),   # nk 16, no bias, fractional mask
]


def make_case(dt, B, S, D, V, bias, mk, seed=0):
    g = torch.Generator().manual_seed(seed)
    dtype = DTYPES[dt]
    H = torch.randn(B, S, D, generator=g).to(dtype)
    W = (torch.randn(V, D, generator=g) * (1.0 / D ** 0.5)).to(dtype)
    b = (torch.randn(V, generator=g) * 0.1 - 0.2).to(dtype) if bias else None
    lens = torch.randint(1, S + 1, (B,), generator=g)
    pad = torch.arange(S)[None] < lens[:, None]
    if mk == "int64":
        m = pad.long()
    elif mk == "int32":
        m = pad.int()
    elif mk == "bool":
        m = pad
    elif mk == "holes":
        m = (torch.rand(B, S, generator=g) < 0.5).long()
        m[0] = 0                                                   # an all-masked row
    elif mk == "gaps":
        m = (pad & ((torch.arange(S)[None] // 256) != 1)).long()  # chunk 1 all masked
        m[1] = 0                                                   # an all-masked row
    elif mk == "frac":
        m = torch.randint(0, 3, (B, S), generator=g).float() * 0.5
    elif mk == "f16":
        m = pad.half()
    elif mk == "bf16":
        m = pad.bfloat16()
    G = torch.rand(B, V, generator=g).to(dtype) * (torch.rand(B, V, generator=g) < 0.3)
    return H, W, b, m, G


@pytest.mark.parametrize("case", CASES, ids=["-".join(map(str, c)) for c in CASES])
def test_random_shapes(case, device):
    say(f"random case {case}")
    H, W, b, m, G = make_case(*case)
    reps, idx, reps32, dH, dW, db = run_fwd_bwd(H, W, b, m, G, device)
    n, bad = check_fwd(H, W, b, m, reps, idx)
    say(f"  checked {n} entries, {bad} near-tie argmax differences")
    check_bwd_isolated(H, W, b, m, G, reps32, idx, dH, dW, db)


@pytest.mark.parametrize("case,grid", PERSISTENT_CASES,
                         ids=[f"{'-'.join(map(str, c))}-G{g}" for c, g in PERSISTENT_CASES])
def test_persistent_schedules(case, grid, device, monkeypatch):
    say(f"random case {case} with {grid} forward workgroups")
    monkeypatch.setenv("SPARTON_FWD_GRID", str(grid))
    H, W, b, m, G = make_case(*case)
    reps, idx, reps32, dH, dW, db = run_fwd_bwd(H, W, b, m, G, device)
    n, bad = check_fwd(H, W, b, m, reps, idx)
    say(f"  checked {n} entries, {bad} near-tie argmax differences")
    check_bwd_isolated(H, W, b, m, G, reps32, idx, dH, dW, db)


def sample_cols(V, n=1024, tail=64, seed=0):
    g = torch.Generator().manual_seed(seed)
    cols = torch.randperm(V, generator=g)[:n]
    return torch.unique(torch.cat([cols, torch.arange(max(0, V - tail), V)]))


@pytest.mark.parametrize("cfg,prec", [(1, "highest"), (1, "high"), (2, None), (3, None), (4, None),
                                      (5, None)])
def test_baseline_config_full_size(cfg, prec, device):
    """Each BASELINE config at full size. Config 1 (fp32) runs under torch's 'highest' (exact
    fp32 MFMAs) and 'high' (the bf16 hi/lo split kernel, the bench default) matmul precision,
    every column against the CPU oracle. Configs 2-5: every (b, v) of reps and argmax against
    float64 library GEMMs on the GPU, every dW row against the identity dW = G'^T H[b, I] on
    the GPU, dH in full against the CPU oracle, and the fp64 oracle on sampled columns."""
    w = WORKLOADS[cfg]
    say(f"config {cfg} {w.name} B={w.B} S={w.S} D={w.D} V={w.V} {w.dtype} precision={prec}")
    inp = make_inputs(w)
    H, W, b, m, G = inp.hidden, inp.weight, inp.bias, inp.mask, inp.grad
    old_prec = torch.get_float32_matmul_precision()
    if prec is not None:
        torch.set_float32_matmul_precision(prec)
    try:
        reps, idx, reps32, dH, dW, db = run_fwd_bwd(H, W, b, m, G, device)
    finally:
        torch.set_float32_matmul_precision(old_prec)
    split = prec == "high"
    cols = None if cfg == 1 else sample_cols(w.V)
    n, bad = check_fwd(H, W, b, m, reps, idx, cols, split=split)
    say(f"  fwd (oracle): checked {n} entries, {bad} near-tie argmax differences")
    if cfg != 1:
        torch.set_float32_matmul_precision("highest")
        try:
            n, bad = check_fwd_full_gpu(H.to(device), W.to(device), None if b is None else b.to(device),
                                        m.to(device), reps, idx)
        finally:
            torch.set_float32_matmul_precision(old_prec)
        say(f"  fwd (every column, fp64 GEMM on the GPU): checked {n} entries, {bad} near-tie "
            f"argmax differences")
        worst = check_dw_identity_gpu(G.to(device), reps32, idx, H.to(device), m.to(device), dW)
        say(f"  dW (every row, identity on the GPU): worst error {worst:.3f} of its bound")
    # Backward: dH in full, dW/dbias on the sampled rows (all rows for config 1).
    reps_c, idx_c = reps32.cpu(), idx.cpu()
    rH, _, rb = oracle.fused_bwd_ref(G, reps_c, idx_c, H, W, b is not None, m, with_dW=False)
    torch.testing.assert_close(dH.cpu().to(F64), rH, **BWD_TOL)
    if cols is None:
        cols = torch.arange(w.V)
    _, rW, _ = oracle.fused_bwd_ref(G[:, cols], reps_c[:, cols], idx_c[:, cols], H, W[cols],
                                      b is not None, m)
    torch.testing.assert_close(dW[cols.to(device)].cpu().to(F64), rW, **BWD_TOL)
    if b is not None:
        torch.testing.assert_close(db.cpu().to(F64), rb, **BWD_TOL)
    # Size-independent identities over every row, with a library GEMM on the GPU:
    # sum_s dH[b,s,:] == G' W  and  dbias == sum_b G'.
    gp = oracle.grad_coeff(G, reps_c, idx_c, m, acc=torch.float32).to(device)
    Wf = W.to(device).float()
    torch.testing.assert_close(dH.sum(1), gp @ Wf, rtol=1e-3, atol=1e-4)
    if b is not None:
        torch.testing.assert_close(db, gp.sum(0), rtol=1e-4, atol=1e-5)
    say(f"  bwd: nnz={int((gp != 0).sum())} ok")


def test_deterministic_repeat(device):
    w = WORKLOADS[2]
    say("determinism, config 2 twice")
    inp = make_inputs(w).to(device)
    outs = []
    for _ in range(2):
        r, i, r32 = torch.ops.sparton.fused_sparton_fwd_train(inp.hidden, inp.weight, inp.bias, inp.mask)
        dh, dw, db = torch.ops.sparton.fused_sparton_bwd(inp.grad, r32, i, inp.hidden, inp.weight,
                                                         inp.bias, inp.mask)
        outs.append([t.clone() for t in (r, i, r32, dh, dw, db)])
    torch.cuda.synchronize()
    for a, c in zip(*outs):
        assert torch.equal(a, c)


@pytest.mark.parametrize("case", [
    ("bf16", 32, 256, 768, 30522, True, "int64"),   # the headline shape
    ("fp16", 8, 512, 768, 9000, True, "holes"),
    ("fp32", 16, 70, 132, 900, False, "frac"),
    ("bf16", 37, 40, 256, 700, True, "int64"),      # many short rows
], ids=lambda c: "-".join(map(str, c)))
def test_backward_paths_agree_bitwise(case, device, monkeypatch):
    """The fused backward (entries compacted by the dW kernel) and the five-kernel one
    (count, scan, scatter; with either dH load-group size) sum every gradient in the same
    order: bitwise equal. (Shapes
    where the fused path is taken: >= 64 row ranges, and >= 1024 rows, so that the
    five-kernel path also gives each dH row one wave.)"""
    say(f"backward paths, case {case}")
    H, W, b, m, G = make_case(*case)
    Hd, Wd, md, Gd = H.to(device), W.to(device), m.to(device), G.to(device)
    bd = None if b is None else b.to(device)
    _, idx, reps32 = torch.ops.sparton.fused_sparton_fwd_train(Hd, Wd, bd, md)
    fused = [t.clone() for t in torch.ops.sparton.fused_sparton_bwd_train(Gd, reps32, idx, Hd, Wd, bd, md)]
    monkeypatch.setenv("SPARTON_BWD_PATH", "five")
    five = [t.clone() for t in torch.ops.sparton.fused_sparton_bwd_train(Gd, reps32, idx, Hd, Wd, bd, md)]
    monkeypatch.setenv("SPARTON_BWD_DH_LONG", "1")  # the large-vocabulary load groups
    five_long = torch.ops.sparton.fused_sparton_bwd_train(Gd, reps32, idx, Hd, Wd, bd, md)
    torch.cuda.synchronize()
    for a, c, d in zip(fused, five, five_long):
        assert torch.equal(a, c) and torch.equal(a, d)


@pytest.mark.parametrize("case", [
    ("bf16", 32, 256, 768, 30522, True, "int64"),   # the headline shape
    ("fp16", 8, 512, 768, 9000, False, "holes"),
    ("fp32", 16, 70, 132, 900, True, "frac"),
    ("bf16", 20, 64, 1280, 3000, True, "int64"),    # two-group batches (bf16 rows past 768)
], ids=lambda c: "-".join(map(str, c)))
def test_backward_hot_rows(case, device, monkeypatch):
    """Rows that win most vocab ids (position 0 scaled up, like a [CLS] token): the fused
    dH workgroup then shares the hot row's batches among its waves. Shared, per-row and
    the automatic choice are bitwise equal, equal to the five-kernel path, and match
    the oracle."""
    say(f"hot dH rows, case {case}")
    H, W, b, m, G = make_case(*case)
    H[:, 0, :] *= 3.0
    Hd, Wd, md, Gd = H.to(device), W.to(device), m.to(device), G.to(device)
    bd = None if b is None else b.to(device)
    _, idx, reps32 = torch.ops.sparton.fused_sparton_fwd_train(Hd, Wd, bd, md)
    runs = {}
    for mode in ("0", "1000", None):
        if mode is None:
            monkeypatch.delenv("SPARTON_BWD_SHARE", raising=False)
        else:
            monkeypatch.setenv("SPARTON_BWD_SHARE", mode)
        runs[mode] = [t.clone() for t in torch.ops.sparton.fused_sparton_bwd(Gd, reps32, idx, Hd, Wd, bd, md)]
    monkeypatch.setenv("SPARTON_BWD_PATH", "five")
    five = torch.ops.sparton.fused_sparton_bwd(Gd, reps32, idx, Hd, Wd, bd, md)
    torch.cuda.synchronize()
    hot = int(torch.bincount(idx[:1].flatten().long().cpu()).max())
    say(f"  row 0's most-won position holds {hot} vocab ids")
    for out in list(runs.values())[1:] + [five]:
        for a, c in zip(runs["0"], out):
            assert (a is None and c is None) or torch.equal(a, c)
    dH, dW, db = runs[None]
    check_bwd_isolated(H, W, b, m, G, reps32, idx, dH, dW, db)


@pytest.mark.parametrize("case", [
    ("bf16", 4, 64, 64, 70000, True, "int64"),      # V > 65536: the five-kernel path
    ("fp32", 8, 100, 96, 8000, False, "int64"),     # five-kernel path forced
    ("fp16", 4, 50, 1280, 12000, True, "int64"),    # five 256-column slices per row
], ids=lambda c: "-".join(map(str, c)))
def test_backward_hot_rows_five_kernel(case, device, monkeypatch):
    """Rows with more than 128 entries (position 0 scaled up) on the five-kernel path go to
    bwd_dh_hot_kernel, whose workgroup shares a row's batches: bitwise the same dH as one
    wave per row (SPARTON_BWD_HOT_MIN set past every row), and the oracle's."""
    say(f"hot dH rows on the five-kernel path, case {case}")
    H, W, b, m, G = make_case(*case)
    H[:, 0, :] *= 3.0
    Hd, Wd, md, Gd = H.to(device), W.to(device), m.to(device), G.to(device)
    bd = None if b is None else b.to(device)
    monkeypatch.setenv("SPARTON_BWD_PATH", "five")
    _, idx, reps32 = torch.ops.sparton.fused_sparton_fwd_train(Hd, Wd, bd, md)
    hot = [t.clone() for t in torch.ops.sparton.fused_sparton_bwd(Gd, reps32, idx, Hd, Wd, bd, md)]
    monkeypatch.setenv("SPARTON_BWD_HOT_MIN", str(2 ** 30))
    plain = torch.ops.sparton.fused_sparton_bwd(Gd, reps32, idx, Hd, Wd, bd, md)
    torch.cuda.synchronize()
    act = (Gd != 0) & (reps32 > 0)
    cnt = torch.zeros(H.shape[0], H.shape[1], dtype=torch.int64, device=device)
    cnt.scatter_add_(1, idx.long(), act.long())
    n_hot = int((cnt > 128).sum())
    say(f"  {n_hot} rows with more than 128 entries (largest {int(cnt.max())})")
    assert n_hot > 0
    for a, c in zip(hot, plain):
        assert (a is None and c is None) or torch.equal(a, c)
    check_bwd_isolated(H, W, b, m, G, reps32, idx, *hot)


def test_graph_capture_replays(device):
    """Forward and backward captured into one HIP graph (all of their kernels and workspace
    allocations) replay to the eager results, bitwise, with eager work and synchronizations
    between the replays."""
    say("graph capture of fwd + bwd, config 3, 3 replays")
    inp = make_inputs(WORKLOADS[3]).to(device)
    H, W, b, m, G = inp.hidden, inp.weight, inp.bias, inp.mask, inp.grad

    def step():
        r, i, r32 = torch.ops.sparton.fused_sparton_fwd_train(H, W, b, m)
        return (r, i, r32) + tuple(torch.ops.sparton.fused_sparton_bwd_train(G, r32, i, H, W, b, m))

    eager = [t.clone() for t in step()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step()
    for k in range(3):
        graph.replay()
        torch.cuda.synchronize()
        _ = (H.float().sum() + W.float().sum()).item()  # eager work between replays
        for a, e in zip(out, eager):
            assert torch.equal(a, e), f"replay {k}"


@pytest.mark.parametrize("cfg", [2, 3])
def test_training_backward_is_fp32_rounded_once(cfg, device):
    """fused_sparton_bwd_train writes each gradient in the input dtype, rounded once from
    the same fp32 sum the fp32 op returns: bitwise equal to that output's cast."""
    w = WORKLOADS[cfg]
    say(f"bwd_train vs bwd, config {cfg}")
    inp = make_inputs(w).to(device)
    r, i, r32 = torch.ops.sparton.fused_sparton_fwd_train(inp.hidden, inp.weight, inp.bias, inp.mask)
    f = torch.ops.sparton.fused_sparton_bwd(inp.grad, r32, i, inp.hidden, inp.weight, inp.bias, inp.mask)
    t = torch.ops.sparton.fused_sparton_bwd_train(inp.grad, r32, i, inp.hidden, inp.weight, inp.bias,
                                                 inp.mask)
    for a, c in zip(t, f):
        assert a.dtype == w.dtype
        assert torch.equal(a, c.to(w.dtype))


def test_encode_equals_training_forward(device):
    say("encode vs fwd, config 3 shape")
    inp = make_inputs(WORKLOADS[3]).to(device)
    r, _ = torch.ops.sparton.fused_sparton_fwd(inp.hidden, inp.weight, inp.bias, inp.mask)
    e = torch.ops.sparton.fused_sparton_encode(inp.hidden, inp.weight, inp.bias, inp.mask)
    assert torch.equal(r, e)
    head = sparton.SpartonHead(inp.weight.shape[0], inp.weight.shape[1], use_bias=True).to(device)
    with torch.no_grad():
        head.weight.copy_(inp.weight.float())
        head.bias.copy_(inp.bias.float())
        out = head.to(torch.float16)(inp.hidden, inp.mask)
    assert torch.equal(out, e)


def test_no_bsv_allocation(device):
    w = WORKLOADS[2]
    say("peak memory, config 2")
    inp = make_inputs(w).to(device)
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    r, i, r32 = torch.ops.sparton.fused_sparton_fwd_train(inp.hidden, inp.weight, inp.bias, inp.mask)
    dh, dw, db = torch.ops.sparton.fused_sparton_bwd(inp.grad, r32, i, inp.hidden, inp.weight, inp.bias, inp.mask)
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated() - base
    bsv = w.B * w.S * w.V * 2
    say(f"  peak extra {peak / 2**20:.1f} MiB vs [B,S,V] bf16 {bsv / 2**20:.1f} MiB")
    outputs = (w.B * w.V * 10 + w.B * w.S * w.D * 4 + w.V * w.D * 4 + w.V * 4)
    assert peak < bsv / 2
    assert peak <= outputs + _lib.load().sparton_bwd_workspace_bytes(w.B, w.S, w.D, w.V) + (8 << 20)


@pytest.mark.parametrize("use_bias", [True, False])
def test_head_autograd_matches_torch_head(use_bias, device):
    """End to end through SpartonHead + autograd vs the repo's torch head in fp32."""
    say(f"SpartonHead autograd vs torch head, bias={use_bias}")
    B, S, D, V = 4, 96, 128, 3000
    g = torch.Generator().manual_seed(5)
    H = torch.randn(B, S, D, generator=g).bfloat16()
    dec = torch.nn.Linear(D, V, bias=use_bias)
    with torch.no_grad():
        dec.weight.copy_(torch.randn(V, D, generator=g) * 0.05)
        if use_bias:
            dec.bias.copy_(torch.randn(V, generator=g) * 0.1 - 0.2)
    dec = dec.bfloat16()
    Wc = dec.weight.detach().clone()
    bc = dec.bias.detach().clone() if use_bias else None
    lens = torch.randint(8, S + 1, (B,), generator=g)
    m = (torch.arange(S)[None] < lens[:, None]).long()
    G = torch.rand(B, V, generator=g).bfloat16()
    # torch head in fp32 on the same rounded values (CPU)
    Hr = H.float().requires_grad_()
    Wr = Wc.float().requires_grad_()
    br = bc.float().requires_grad_() if use_bias else None
    ref = oracle.torch_head(Hr, Wr, br, m)
    ref.backward(G.float())
    # SpartonHead tied to the decoder, as training/model.py:77-80 does
    decd = dec.to(device)
    head = sparton.SpartonHead(decd.out_features, decd.in_features, use_bias=use_bias).to(device)
    head.tie_weights(decd)
    Hd = H.to(device).requires_grad_()
    out = head(Hd, m.to(device))
    out.backward(G.to(device))
    torch.testing.assert_close(out.detach().cpu().float(), ref.detach(), **FWD_TOL)
    # rows an argmax near-tie could move are excluded from the gradient comparison
    _, I, _ = oracle.fused_fwd_ref(H, Wc, bc, m)
    _, idx = torch.ops.sparton.fused_sparton_fwd(Hd.detach(), decd.weight.detach(),
                                                 decd.bias.detach() if use_bias else None, m.to(device))
    idx = idx.cpu().long()
    moved = idx != I
    say(f"  near-tie moved entries: {int(moved.sum())}")
    vok = ~moved.any(0)
    hok = torch.ones(B, S, dtype=torch.bool)
    for bb, vv in moved.nonzero().tolist():
        hok[bb, I[bb, vv]] = False
        hok[bb, idx[bb, vv]] = False
    torch.testing.assert_close(decd.weight.grad.cpu().float()[vok], Wr.grad[vok], **FWD_TOL)
    torch.testing.assert_close(Hd.grad.cpu().float()[hok], Hr.grad[hok], **FWD_TOL)
    if use_bias:
        torch.testing.assert_close(decd.bias.grad.cpu().float()[vok], br.grad[vok], **FWD_TOL)
    assert Hd.grad.dtype == torch.bfloat16 and decd.weight.grad.dtype == torch.bfloat16


def test_edge_cases(device):
    say("edge cases")
    # empty sequence: every rep is 0 and every index 0
    H = torch.zeros(2, 0, 16, dtype=torch.bfloat16, device=device)
    W = torch.randn(40, 16, device=device).bfloat16()
    m = torch.zeros(2, 0, dtype=torch.long, device=device)
    r, i = torch.ops.sparton.fused_sparton_fwd(H, W, None, m)
    assert torch.all(r == 0) and torch.all(i == 0)
    # D == 0: x = bias * mask, the first valid position wins every positive column
    H0 = torch.zeros(2, 5, 0, dtype=torch.bfloat16)
    W0 = torch.zeros(40, 0, dtype=torch.bfloat16)
    b0 = (torch.randn(40) * 0.5).bfloat16()
    m0 = torch.tensor([[0, 1, 1, 0, 0], [1, 1, 1, 1, 1]])
    r0, i0 = torch.ops.sparton.fused_sparton_fwd(H0.to(device), W0.to(device), b0.to(device), m0.to(device))
    M0, I0, ref0 = oracle.fused_fwd_ref(H0, W0, b0, m0)
    torch.testing.assert_close(r0.cpu().to(F64), ref0, **FWD_TOL)
    assert torch.equal(i0.cpu().long(), I0)
    # non-multiple-of-8 hidden size goes through SpartonHead's zero padding
    B, S, D, V = 2, 9, 20, 50
    H = torch.randn(B, S, D).bfloat16()
    head = sparton.SpartonHead(V, D, use_bias=True)
    m = torch.ones(B, S, dtype=torch.long)
    with torch.no_grad():
        ref = oracle.torch_head(H.float(), head.weight.bfloat16().float(), head.bias.bfloat16().float(), m)
        out = head.to(device).bfloat16()(H.to(device), m.to(device))
    torch.testing.assert_close(out.cpu().float(), ref, **FWD_TOL)
    # a mask on another dtype / non-contiguous hidden
    H2 = torch.randn(5, 3, 32, device=device).bfloat16().transpose(0, 1)   # [3,5,32] non-contiguous
    W2 = torch.randn(70, 32, device=device).bfloat16() * 0.2
    m2 = torch.ones(3, 5, dtype=torch.bool, device=device)
    r2, i2 = torch.ops.sparton.fused_sparton_fwd(H2, W2, None, m2)
    M, I, ref2 = oracle.fused_fwd_ref(H2.cpu(), W2.cpu(), None, m2.cpu())
    torch.testing.assert_close(r2.cpu().to(F64), ref2, **FWD_TOL)


@pytest.mark.parametrize("dt,D", [("bf16", 24), ("fp16", 8), ("fp32", 12), ("bf16", 72)])
def test_reads_stay_inside_rows(dt, D, device):
    """Rows shorter than (or not a multiple of) one 128-byte K slab: the bytes right
    after H and W are NaN, so a load past a row end -- which would poison a logit with
    NaN * 0 -- shows up as a wrong max. The last position of each batch row is made
    the argmax of many columns, so its row (the one next to the NaNs) must be used."""
    say(f"NaN-fenced H and W, {dt} D={D}")
    dtype = DTYPES[dt]
    B, S, V = 3, 9, 300
    g = torch.Generator().manual_seed(7)
    H = torch.randn(B, S, D, generator=g)
    H[:, -1] *= 4.0
    W = (torch.randn(V, D, generator=g) * 0.3).to(dtype)
    H = H.to(dtype)
    b = (torch.randn(V, generator=g) * 0.1).to(dtype)
    m = torch.ones(B, S, dtype=torch.long)
    m[1, 5:] = 0
    pad = 256
    Hbuf = torch.full((B * S * D + pad,), float("nan"), dtype=dtype, device=device)
    Wbuf = torch.full((V * D + pad,), float("nan"), dtype=dtype, device=device)
    Hd = Hbuf[: B * S * D].view(B, S, D)
    Wd = Wbuf[: V * D].view(V, D)
    Hd.copy_(H)
    Wd.copy_(W)
    reps, idx = torch.ops.sparton.fused_sparton_fwd(Hd, Wd, b.to(device), m.to(device))
    torch.cuda.synchronize()
    assert torch.isnan(Hbuf[B * S * D:]).all() and torch.isnan(Wbuf[V * D:]).all()
    n, bad = check_fwd(H, W, b, m, reps, idx)
    say(f"  checked {n} entries, {bad} near-tie argmax differences")


def test_fwd_profile_entry_point_matches_fwd(device):
    """sparton_fwd_profile does the same work as sparton_fwd and reports the main
    kernel's device time."""
    import ctypes
    say("sparton_fwd_profile vs sparton_fwd")
    H, W, b, m, _ = make_case("bf16", 3, 77, 64, 1000, True, "int64")
    Hd, Wd, bd, md = H.to(device), W.to(device), b.to(device), m.to(device)
    r_ref, i_ref, r32_ref = torch.ops.sparton.fused_sparton_fwd_train(Hd, Wd, bd, md)
    L = _lib.load()
    B, S, D = H.shape
    V = W.shape[0]
    dt = _lib.DTYPE_CODE[H.dtype]
    reps = torch.empty_like(r_ref)
    idx = torch.empty_like(i_ref)
    r32 = torch.empty_like(r32_ref)
    nbytes = int(L.sparton_fwd_workspace_bytes(B, S, D, V, dt))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    ms = ctypes.c_float(-1.0)
    rc = L.sparton_fwd_profile(Hd.data_ptr(), Wd.data_ptr(), bd.data_ptr(), md.data_ptr(),
                               _lib.MASK_CODE[md.dtype], reps.data_ptr(), idx.data_ptr(),
                               r32.data_ptr(), B, S, D, V, dt, ws.data_ptr(), nbytes,
                               torch.cuda.current_stream().cuda_stream, ctypes.byref(ms))
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(reps, r_ref) and torch.equal(idx, i_ref) and torch.equal(r32, r32_ref)
    assert 0.0 < ms.value < 1000.0


def test_autocast_policy(device):
    say("autocast bf16 with fp32 parameters")
    B, S, D, V = 2, 64, 64, 500
    head = sparton.SpartonHead(V, D, use_bias=True).to(device)
    H = torch.randn(B, S, D, device=device)
    m = torch.ones(B, S, dtype=torch.long, device=device)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = head(H, m)
    assert out.dtype == torch.bfloat16
    ref = oracle.torch_head(H.cpu().bfloat16().double(), head.weight.detach().cpu().bfloat16().double(),
                            head.bias.detach().cpu().bfloat16().double(), m.cpu())
    torch.testing.assert_close(out.cpu().double(), ref, **FWD_TOL)


@pytest.mark.parametrize("dt,D,V", [(torch.bfloat16, 60, 700), (torch.float16, 64, 700),
                                    (torch.bfloat16, 40, 70001)])  # V > 65536: five-kernel backward
def test_autocast_fp32_master_gradients(dt, D, V, device):
    """Autocast over fp32 parameters and fp32 hidden states (mixed-precision training):
    the gradients come out in fp32, equal to the oracle's at the kernel's own argmax and
    unrounded reps, and equal, once rounded to the compute dtype, to the plain path's
    (cast the parameters, run the training op, let autograd cast the gradients back)."""
    say(f"autocast {dt} fp32 masters D={D} V={V}")
    B, S = 3, 70
    g = torch.Generator().manual_seed(D)
    head = sparton.SpartonHead(V, D, use_bias=True).to(device)
    H = torch.randn(B, S, D, generator=g).to(device).requires_grad_()
    lens = torch.tensor([70, 33, 5])
    m = (torch.arange(S)[None] < lens[:, None]).long().to(device)
    G = torch.rand(B, V, generator=g).to(dt).to(device)
    with torch.autocast("cuda", dtype=dt):
        out = head(H, m)
    assert out.dtype == dt
    out.backward(G)
    dH, dW, db = H.grad, head.weight.grad, head.bias.grad
    assert dH.dtype == dW.dtype == db.dtype == torch.float32
    # the oracle at the kernel's own argmax and fp32 reps, on the rounded inputs
    pad = (-D) % 8
    Hl = F.pad(H.detach().to(dt), (0, pad))
    Wl = F.pad(head.weight.detach().to(dt), (0, pad))
    bl = head.bias.detach().to(dt)
    reps, idx, reps32 = torch.ops.sparton.fused_sparton_fwd_train(Hl, Wl, bl, m)
    assert torch.equal(reps, out.detach())
    rH, rW, rb = oracle.fused_bwd_ref(G.cpu(), reps32.cpu(), idx.cpu(), Hl.cpu(), Wl.cpu(), True, m.cpu())
    torch.testing.assert_close(dH.cpu().to(F64), rH[..., :D], **BWD_TOL)
    torch.testing.assert_close(dW.cpu().to(F64), rW[:, :D], **BWD_TOL)
    torch.testing.assert_close(db.cpu().to(F64), rb, **BWD_TOL)
    # the plain path: 16-bit gradients rounded once from the same fp32 sums
    hp = H.detach().to(dt).requires_grad_()
    wp = head.weight.detach().to(dt).requires_grad_()
    bp = head.bias.detach().to(dt).requires_grad_()
    rp, _, _ = torch.ops.sparton.fused_sparton_fwd_train(F.pad(hp, (0, pad)), F.pad(wp, (0, pad)), bp, m)
    rp.backward(G)
    assert torch.equal(dW.to(dt), wp.grad) and torch.equal(db.to(dt), bp.grad)
    assert torch.equal(dH.to(dt), hp.grad)


def test_opcheck_and_compile(device):
    say("opcheck + torch.compile(aot_eager)")
    B, S, D, V = 2, 16, 32, 100
    H = torch.randn(B, S, D, device=device).bfloat16()
    W = (torch.randn(V, D, device=device) * 0.2).bfloat16()
    b = (torch.randn(V, device=device) * 0.1).bfloat16()
    m = torch.ones(B, S, dtype=torch.long, device=device)
    torch.library.opcheck(torch.ops.sparton.fused_sparton_fwd.default, (H, W, b, m),
                          test_utils=("test_schema", "test_faketensor"))
    # with inputs that require grad, the autograd registration is checked as well
    Hg, Wg, bg = (t.clone().requires_grad_() for t in (H, W, b))
    for op in (torch.ops.sparton.fused_sparton_fwd.default, torch.ops.sparton.fused_sparton_fwd_train.default):
        torch.library.opcheck(op, (Hg, Wg, bg, m), test_utils=("test_autograd_registration",))
    head = sparton.SpartonHead(V, D, use_bias=True).to(device).bfloat16()

    def f(h, mm):
        return head(h, mm).float().sum()

    cf = torch.compile(f, backend="aot_eager", fullgraph=True)
    Hc = H.clone().requires_grad_()
    y = cf(Hc, m)
    y.backward()
    He = H.clone().requires_grad_()
    ye = f(He, m)
    ye.backward()
    assert torch.equal(y, ye) and torch.equal(Hc.grad, He.grad)


@pytest.mark.parametrize("case", [
    ("fp32", 2, 32, 768, 3000, True, "int64"),     # 64 rows: 8 waves per dH row
    ("bf16", 3, 100, 256, 2000, True, "holes"),    # 300 rows: 4 waves per row
    ("fp16", 1, 700, 64, 500, False, "frac"),      # 700 rows: 2 waves per row
], ids=lambda c: "-".join(map(str, c)))
def test_backward_few_rows_split(case, device, monkeypatch):
    """Few dH rows: the five-kernel path splits each row's entries over several waves and
    adds their partial rows in wave order (SPARTON_BWD_FEW=0 keeps batches of at most 64 rows
    on it too). Against the oracle, and bitwise repeatable."""
    say(f"backward few rows, case {case}")
    monkeypatch.setenv("SPARTON_BWD_FEW", "0")
    H, W, b, m, G = make_case(*case)
    Hd, Wd, md, Gd = H.to(device), W.to(device), m.to(device), G.to(device)
    bd = None if b is None else b.to(device)
    _, idx, reps32 = torch.ops.sparton.fused_sparton_fwd_train(Hd, Wd, bd, md)
    outs = [[t.clone() for t in torch.ops.sparton.fused_sparton_bwd(Gd, reps32, idx, Hd, Wd, bd, md)]
            for _ in range(2)]
    torch.cuda.synchronize()
    for a, c in zip(*outs):
        assert torch.equal(a, c)
    check_bwd_isolated(H, W, b, m, G, reps32, idx, *outs[0])



FEW_ROW_CASES = [
    ("fp32", 2, 32, 768, 30522, True, "int64"),    # config 1's shape: W read once for both rows
    ("bf16", 1, 64, 1024, 5000, False, "frac"),    # one batch row of 64 positions, no bias
    ("fp16", 64, 1, 128, 3000, True, "bool"),      # 64 batch rows of one position
    ("fp32", 3, 20, 72, 2000, True, "holes"),      # a partial 256-column slice, masked holes
    ("bf16", 2, 16, 4096, 3000, True, "int64"),    # 16 column slices
    ("fp16", 5, 7, 264, 777, True, "gaps"),        # ragged everything
]


@pytest.mark.parametrize("case", FEW_ROW_CASES, ids=lambda c: "-".join(map(str, c)))
def test_backward_few_rows_single_w_read(case, device, monkeypatch):
    """At most 64 dH rows: each W row is read once and added into every dH row it serves
    (rows held in registers, per-range partials added in range order). Against the oracle,
    bitwise repeatable, dW and dbias bitwise those of the five-kernel path, dH within fp32
    rounding of it (the two sum in different orders)."""
    say(f"backward few rows, single W read, case {case}")
    H, W, b, m, G = make_case(*case)
    Hd, Wd, md, Gd = H.to(device), W.to(device), m.to(device), G.to(device)
    bd = None if b is None else b.to(device)
    _, idx, reps32 = torch.ops.sparton.fused_sparton_fwd_train(Hd, Wd, bd, md)
    outs = [[None if t is None else t.clone()
             for t in torch.ops.sparton.fused_sparton_bwd(Gd, reps32, idx, Hd, Wd, bd, md)]
            for _ in range(2)]
    monkeypatch.setenv("SPARTON_BWD_FEW", "0")
    other = torch.ops.sparton.fused_sparton_bwd(Gd, reps32, idx, Hd, Wd, bd, md)
    torch.cuda.synchronize()
    for a, c in zip(*outs):
        assert (a is None and c is None) or torch.equal(a, c)
    torch.testing.assert_close(outs[0][0], other[0], **BWD_TOL)
    assert torch.equal(outs[0][1], other[1])
    assert (outs[0][2] is None and other[2] is None) or torch.equal(outs[0][2], other[2])
    if Hd.dtype != torch.float32:
        # gradients in the input dtype: dW and dbias the same bits, dH within one rounding
        tr_other = torch.ops.sparton.fused_sparton_bwd_train(Gd, reps32, idx, Hd, Wd, bd, md)
        monkeypatch.delenv("SPARTON_BWD_FEW")
        tr = torch.ops.sparton.fused_sparton_bwd_train(Gd, reps32, idx, Hd, Wd, bd, md)
        torch.cuda.synchronize()
        assert tr[1].dtype == Hd.dtype and torch.equal(tr[1], tr_other[1])
        assert torch.equal(tr[2], tr_other[2])
        torch.testing.assert_close(tr[0].float(), tr_other[0].float(), rtol=1e-2, atol=1e-6)
    check_bwd_isolated(H, W, b, m, G, reps32, idx, *outs[0])


def _bwd_capi(Gd, reps32, idx, Hd, Wd, md, dH, dW, db):
    """sparton_bwd through the C ABI with any of the three outputs left out (None)."""
    B, S, D = Hd.shape
    V = Wd.shape[0]
    L = _lib.load()
    ws_bytes = int(L.sparton_bwd_workspace_bytes(B, S, D, V))
    ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=Hd.device)
    ptr = lambda t: None if t is None else t.data_ptr()
    Gd = Gd.to(Hd.dtype).contiguous()
    rc = L.sparton_bwd(Gd.data_ptr(), reps32.data_ptr(), _lib.DTYPE_CODE[reps32.dtype],
                       idx.data_ptr(), md.data_ptr(), _lib.MASK_CODE[md.dtype], Hd.data_ptr(),
                       Wd.data_ptr(), ptr(dH), ptr(dW), ptr(db), _lib.DTYPE_CODE[torch.float32],
                       ws.data_ptr(), ws_bytes, B, S, D, V, _lib.DTYPE_CODE[Hd.dtype],
                       torch.cuda.current_stream().cuda_stream)
    assert rc == 0, L.sparton_strerror(rc)


@pytest.mark.parametrize("case", [FEW_ROW_CASES[0], FEW_ROW_CASES[2], FEW_ROW_CASES[5]],
                         ids=lambda c: "-".join(map(str, c)))
def test_backward_few_rows_partial_outputs(case, device):
    """The few-row launch asked for dH with dbias but no dW, and for dH with dW but no
    dbias: the outputs it does write are bitwise those of the full call."""
    say(f"backward few rows, partial outputs, case {case}")
    H, W, b, m, G = make_case(*case)
    Hd, Wd, md, Gd = H.to(device), W.to(device), m.to(device), G.to(device)
    bd = None if b is None else b.to(device)
    _, idx, reps32 = torch.ops.sparton.fused_sparton_fwd_train(Hd, Wd, bd, md)
    B, S, D = Hd.shape
    V = Wd.shape[0]
    f32 = dict(dtype=torch.float32, device=device)
    full = [torch.empty((B, S, D), **f32), torch.empty((V, D), **f32), torch.empty((V,), **f32)]
    _bwd_capi(Gd, reps32, idx, Hd, Wd, md, *full)
    no_dw = [torch.empty((B, S, D), **f32), torch.empty((V,), **f32)]
    _bwd_capi(Gd, reps32, idx, Hd, Wd, md, no_dw[0], None, no_dw[1])
    no_db = [torch.empty((B, S, D), **f32), torch.empty((V, D), **f32)]
    _bwd_capi(Gd, reps32, idx, Hd, Wd, md, no_db[0], no_db[1], None)
    torch.cuda.synchronize()
    assert torch.equal(no_dw[0], full[0]) and torch.equal(no_dw[1], full[2])
    assert torch.equal(no_db[0], full[0]) and torch.equal(no_db[1], full[1])


@pytest.mark.parametrize("case,long_rows", [
    (("fp32", 2, 32, 768, 3000, True, "int64"), False),    # few rows: split dH + dW, one launch
    (("bf16", 3, 100, 256, 2000, False, "holes"), False),  # few rows, no bias
    (("bf16", 8, 160, 1536, 1200, True, "int64"), False),  # 1280 rows, six register passes
    (("fp16", 6, 200, 2048, 3000, True, "frac"), True),    # eight passes, long-row dH groups
], ids=lambda c: "-".join(map(str, c)) if isinstance(c, tuple) else f"long{int(c)}")
def test_backward_dw_in_dh_launch(case, long_rows, device, monkeypatch):
    """On the five-kernel path, dW's workgroups run in the dH launch (few rows, or rows of
    six or more register passes): bitwise the same dH, dW and dbias as a separate dW
    launch (SPARTON_BWD_DW_MERGE=0), and the oracle's."""
    say(f"dW in the dH launch, case {case}, long-row groups {long_rows}")
    H, W, b, m, G = make_case(*case)
    Hd, Wd, md, Gd = H.to(device), W.to(device), m.to(device), G.to(device)
    bd = None if b is None else b.to(device)
    monkeypatch.setenv("SPARTON_BWD_PATH", "five")
    monkeypatch.setenv("SPARTON_BWD_FEW", "0")
    if long_rows:
        monkeypatch.setenv("SPARTON_BWD_DH_LONG", "1")
    _, idx, reps32 = torch.ops.sparton.fused_sparton_fwd_train(Hd, Wd, bd, md)
    merged = [None if t is None else t.clone()
              for t in torch.ops.sparton.fused_sparton_bwd(Gd, reps32, idx, Hd, Wd, bd, md)]
    monkeypatch.setenv("SPARTON_BWD_DW_MERGE", "0")
    apart = torch.ops.sparton.fused_sparton_bwd(Gd, reps32, idx, Hd, Wd, bd, md)
    torch.cuda.synchronize()
    for a, c in zip(merged, apart):
        assert (a is None and c is None) or torch.equal(a, c)
    check_bwd_isolated(H, W, b, m, G, reps32, idx, *merged)


@pytest.mark.parametrize("case", [
    ("bf16", 2, 20000, 64, 320, True, "holes"),     # S > 16384: two dH windows
    ("fp32", 1, 40000, 32, 200, False, "int64"),    # three windows, the last partial
    ("fp16", 20, 20000, 32, 64, True, "gaps"),      # 25000 groups: the three-kernel plan
    ("bf16", 9000, 3, 32, 64, True, "int64"),       # B > 8192: two dH batch chunks
    ("bf16", 33000, 1, 8, 16, True, "holes"),       # B > 32768: two forward launches
    ("bf16", 1, 70000, 16, 64, True, "int64"),      # S > 65536: dW without the 16-bit staging
], ids=lambda c: "-".join(map(str, c)))
def test_long_sequences_and_many_rows(case, device):
    """Shapes past one pass of the kernels: the forward takes any S (and splits B over
    launches of at most 32768 rows); the backward's dH passes run over windows of 16384
    positions and chunks of 8192 batch rows. Against the oracle."""
    say(f"long / many rows, case {case}")
    H, W, b, m, G = make_case(*case)
    reps, idx, reps32, dH, dW, db = run_fwd_bwd(H, W, b, m, G, device)
    n, bad = check_fwd(H, W, b, m, reps, idx)
    say(f"  checked {n} entries, {bad} near-tie argmax differences")
    check_bwd_isolated(H, W, b, m, G, reps32, idx, dH, dW, db)


@pytest.mark.parametrize("case", [
    ("fp32", 2, 32, 768, 30522, True, "int64"),     # config 1: 64 rows
    ("fp32", 3, 40, 256, 1000, True, "holes"),      # 120 rows: four 32-row blocks
    ("fp32", 1, 7, 12, 100, False, "frac"),         # one block, D in one partial slab
    ("fp32", 5, 20, 132, 333, True, "int64"),       # 100 rows, a 16-byte tail slab
    ("fp32", 128, 1, 72, 5000, True, "bool"),       # S = 1: every row its own batch row
    ("fp32", 2, 48, 2048, 2000, False, "int64"),    # 64 full slabs
    ("bf16", 2, 32, 768, 30522, True, "int64"),     # 16-bit, config 2's widths
    ("bf16", 3, 40, 256, 1000, True, "holes"),      # 120 rows: four 32-row blocks
    ("fp16", 1, 7, 24, 100, False, "frac"),         # one block, D in one partial slab
    ("bf16", 128, 1, 72, 5000, True, "bool"),       # S = 1, a 16-byte tail slab
    ("bf16", 2, 48, 4096, 2000, False, "int64"),    # 64 full slabs
], ids=lambda c: "-".join(map(str, c)))
def test_small_batch_path_equals_main_path(case, device, monkeypatch):
    """Batches of B * S <= 128 rows (16-bit ones up to B * S * V = 2^24) take one kernel
    (one wave per 32 vocab columns, all rows, W read once). It sums every logit in the
    main kernel's order and applies the same key order, so reps, argmax and the fp32 reps
    equal the plan / main / fixup path's bitwise; and both match the oracle."""
    say(f"small-batch path vs main path, case {case}")
    H, W, b, m, G = make_case(*case)
    Hd, Wd, md = H.to(device), W.to(device), m.to(device)
    bd = None if b is None else b.to(device)
    small = [t.clone() for t in torch.ops.sparton.fused_sparton_fwd_train(Hd, Wd, bd, md)]
    monkeypatch.setenv("SPARTON_FWD_PATH", "main")
    main = torch.ops.sparton.fused_sparton_fwd_train(Hd, Wd, bd, md)
    torch.cuda.synchronize()
    for a, c in zip(small, main):
        assert torch.equal(a, c)
    n, bad = check_fwd(H, W, b, m, small[0], small[1])
    say(f"  checked {n} entries, {bad} near-tie argmax differences")


SPLIT_CASES = [
    ("fp32", 2, 32, 768, 3000, True, "int64"),     # config 1's rows and width
    ("fp32", 1, 100, 1024, 2000, False, "frac"),   # four 32-row blocks, fractional mask
    ("fp32", 4, 32, 72, 500, True, "holes"),       # 288-byte rows: a 32-byte tail slab
    ("fp32", 3, 40, 4, 300, True, "bool"),         # D = 4: one 16-byte chunk per row
    ("fp32", 2, 48, 2048, 1200, False, "int64"),   # 64 full slabs
]


@pytest.mark.parametrize("case", SPLIT_CASES, ids=lambda c: "-".join(map(str, c)))
def test_fp32_split_precision(case, device):
    """Under torch's 'high' float32 matmul precision, which the reference sets at import
    (sparton_kernel.py:14), small fp32 batches take each product as bf16 hi*hi + hi*lo +
    lo*hi, within 3 * 2^-16 relative of the exact product. Checked against the oracle with
    the tie band widened by that bound, and entry by entry: the fp32 reps against log1p of
    the exact logit at the chosen index,
    |reps - log1p(x)| <= (2^-18 x + (gamma_{D+2} + 3 * 2^-16) * sum|h w + b|) / (1 + x)
    + 2^-23 + 2^-21 log1p(x). 'highest' gives the exact path back (bitwise the main path)."""
    say(f"fp32 split precision, case {case}")
    H, W, b, m, _ = make_case(*case)
    Hd, Wd, md = H.to(device), W.to(device), m.to(device)
    bd = None if b is None else b.to(device)
    prev = torch.get_float32_matmul_precision()
    try:
        torch.set_float32_matmul_precision("high")
        reps, idx, r32 = [t.clone() for t in torch.ops.sparton.fused_sparton_fwd_train(Hd, Wd, bd, md)]
        # the C++ eager op (SpartonHead's path) reads the same setting
        from sparton_amd import _eager
        assert torch.equal(_eager.load().head_encode(Hd, Wd, bd, md), reps)
        torch.set_float32_matmul_precision("highest")
        exact = [t.clone() for t in torch.ops.sparton.fused_sparton_fwd_train(Hd, Wd, bd, md)]
    finally:
        torch.set_float32_matmul_precision(prev)
    torch.cuda.synchronize()
    n, bad = check_fwd(H, W, b, m, reps, idx, split=True)
    say(f"  checked {n} entries, {bad} near-tie argmax differences")
    # the value at the chosen index
    idx_c = idx.cpu().long()
    x = oracle.logit_at(H, W, b, m, idx_c)
    A = oracle.logit_at(H.abs(), W.abs(), None if b is None else b.abs(),
                        m if m.dtype == torch.bool else m.abs(), idx_c)
    D = H.shape[-1]
    r = r32.cpu().to(F64)
    pos = r > 0
    lx = torch.log1p(x.clamp_min(0))
    bound = ((2.0 ** -18 * x.abs() + ((D + 2) * 2.0 ** -24 + 3 * 2.0 ** -16) * A) / (1 + x.clamp_min(0))
             + 2.0 ** -23 + 2.0 ** -21 * lx)
    err = (r - lx).abs()
    assert bool((err[pos] <= bound[pos]).all()), float((err - bound)[pos].max())
    say(f"  max |reps - log1p(x)| = {float(err[pos].max()):.3e}")
    # the exact path is unchanged: bitwise the main kernel's fp32
    main = None
    os.environ["SPARTON_FWD_PATH"] = "main"
    try:
        main = torch.ops.sparton.fused_sparton_fwd_train(Hd, Wd, bd, md)
    finally:
        del os.environ["SPARTON_FWD_PATH"]
    torch.cuda.synchronize()
    for a, c in zip(exact, main):
        assert torch.equal(a, c)
    if D >= 64:  # the split path is a different computation (its values move at 2^-18)
        assert not torch.equal(r32, exact[2])


def test_fp32_split_infinite_entries(device):
    """Infinite entries in H and in W under 'high' (the bf16 hi/lo split kernel): reps and
    argmax equal the exact fp32 path's ('highest'), infinities and NaNs included, as long as
    no product has both operands infinite. A pair holding a non-finite value keeps it in its
    lo part (hi = 0), so only one of the three bf16 products sees the infinity."""
    say("fp32 split mode with infinite entries in H and W")
    g = torch.Generator().manual_seed(21)
    B, S, D, V = 2, 32, 768, 3000
    H = torch.randn(B, S, D, generator=g)
    W = torch.randn(V, D, generator=g) * 0.02
    b = torch.randn(V, generator=g) * 0.02
    m = torch.ones(B, S, dtype=torch.long)
    m[1, 20:] = 0
    H[0, 5, 17] = float("inf")
    H[1, 3, 400] = float("-inf")
    W[7, 100] = float("-inf")
    W[2999, 767] = float("inf")
    Hd, Wd, bd, md = H.to(device), W.to(device), b.to(device), m.to(device)
    prev = torch.get_float32_matmul_precision()
    try:
        torch.set_float32_matmul_precision("high")
        split = [t.clone() for t in torch.ops.sparton.fused_sparton_fwd_train(Hd, Wd, bd, md)]
        torch.set_float32_matmul_precision("highest")
        exact = [t.clone() for t in torch.ops.sparton.fused_sparton_fwd_train(Hd, Wd, bd, md)]
    finally:
        torch.set_float32_matmul_precision(prev)
    torch.cuda.synchronize()
    r_s, r_e = split[2].cpu(), exact[2].cpu()
    nonfinite = ~torch.isfinite(r_e)
    say(f"  {int(nonfinite.sum())} non-finite reps in the exact path, "
        f"{int(torch.isinf(r_e).sum())} infinite")
    assert int(torch.isinf(r_e).sum()) > 100
    assert torch.equal(nonfinite, ~torch.isfinite(r_s))
    assert torch.equal(r_s[nonfinite].isnan(), r_e[nonfinite].isnan())
    assert torch.equal(r_s[torch.isinf(r_e)], r_e[torch.isinf(r_e)])
    assert torch.equal(split[1].cpu()[nonfinite], exact[1].cpu()[nonfinite])
    fin = ~nonfinite
    torch.testing.assert_close(r_s[fin].double(), r_e[fin].double(), **FWD_TOL)


@pytest.mark.parametrize("dt", [1, 2])
def test_mfma_probe_reports_cycles(dt, device):
    """sparton_mfma_probe (the measurement kernel bench.py reports as mfma_ceiling) runs on
    every CU and reports positive cycle and real-time counts at a plausible shader clock."""
    say(f"mfma probe, dtype code {dt}")
    L = _lib.load()
    grid = torch.cuda.get_device_properties(0).multi_processor_count
    out = torch.empty(grid * 256, dtype=torch.float32, device=device)
    clk = torch.zeros(grid * 2, dtype=torch.int64, device=device)
    rc = L.sparton_mfma_probe(dt, grid, 50, out.data_ptr(), clk.data_ptr(),
                              torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    c = clk.view(grid, 2).double().cpu()
    assert bool((c > 0).all())
    mhz = c[:, 0] / (c[:, 1] / 100.0)
    assert bool(((mhz > 300) & (mhz < 3500)).all()), mhz
    assert bool(torch.isfinite(out).all())
    assert L.sparton_mfma_probe(0, grid, 50, out.data_ptr(), clk.data_ptr(), None) == -1

@pytest.mark.parametrize("cfg,use_bias", [(2, True), (3, False)])
def test_reference_op_autograd(cfg, use_bias, device):
    """Backprop through torch.ops.sparton.fused_sparton_fwd, the route the reference's
    SpartonHead.forward takes (sparton_kernel.py:744 and register_autograd at :707): its
    backward calls sparton::fused_sparton_bwd with the op's rounded scores (:701-705), which
    returns fp32 gradients (:676-678); autograd casts them to each input's dtype. Checked
    bitwise against that fp32 op's output cast once, and against the oracle's closed form at
    the op's own reps and argmax."""
    w = WORKLOADS[cfg]
    say(f"reference-op autograd, config {cfg} {w.name} bias={use_bias}")
    inp = make_inputs(w)
    H, W, m, G = inp.hidden, inp.weight, inp.mask, inp.grad
    b = inp.bias if use_bias else None
    Hd, Wd = H.to(device).requires_grad_(), W.to(device).requires_grad_()
    bd = b.to(device).requires_grad_() if b is not None else None
    md, Gd = m.to(device), G.to(device)
    reps, idx = torch.ops.sparton.fused_sparton_fwd(Hd, Wd, bd, md)
    assert idx.dtype == torch.int32 and not idx.requires_grad and reps.dtype == w.dtype
    reps.backward(Gd)
    torch.cuda.synchronize()
    assert Hd.grad.dtype == Wd.grad.dtype == w.dtype
    if b is not None:
        assert bd.grad.dtype == w.dtype
    # the registered backward is the fp32 reference op at the rounded reps, cast once
    dH32, dW32, db32 = torch.ops.sparton.fused_sparton_bwd(Gd, reps.detach(), idx, Hd.detach(),
                                                           Wd.detach(), None if bd is None else bd.detach(), md)
    assert dH32.dtype == dW32.dtype == torch.float32
    assert torch.equal(Hd.grad, dH32.to(w.dtype)) and torch.equal(Wd.grad, dW32.to(w.dtype))
    if b is not None:
        assert torch.equal(bd.grad, db32.to(w.dtype))
    else:
        assert db32.numel() == 0
    # the fp32 gradients against the oracle at the op's own reps and argmax
    reps_c, idx_c = reps.detach().cpu(), idx.cpu()
    rH, _, rb = oracle.fused_bwd_ref(G, reps_c, idx_c, H, W, b is not None, m, with_dW=False)
    torch.testing.assert_close(dH32.cpu().to(F64), rH, **BWD_TOL)
    cols = sample_cols(w.V)
    _, rW, _ = oracle.fused_bwd_ref(G[:, cols], reps_c[:, cols], idx_c[:, cols], H, W[cols],
                                    b is not None, m)
    torch.testing.assert_close(dW32[cols.to(device)].cpu().to(F64), rW, **BWD_TOL)
    if b is not None:
        torch.testing.assert_close(db32.cpu().to(F64), rb, **BWD_TOL)
    say(f"  nnz={int((G != 0).sum())} ok")


def test_reps_value_truncation_bound(device):
    """The kernel's max keeps each logit with its 5 low mantissa bits cleared (the row index
    takes them), so in fp32 reps = log1p(M') with M - M' <= 2^-18 M, always rounding down,
    plus the fp32 accumulation error and the kernel's log1p (a few ulp). Bounded here on an
    fp32 case, entry by entry:
    |reps - log1p(M)| <= (2^-18 M + gamma_{D+2} * sum|h w + b| at the oracle's argmax) / (1 + M)
    + 2^-23 + 2^-21 log1p(M)."""
    say("fp32 reps value bound")
    H, W, b, m, _ = make_case("fp32", 4, 200, 384, 3000, True, "int64", seed=3)
    reps, idx, r32 = torch.ops.sparton.fused_sparton_fwd_train(H.to(device), W.to(device), b.to(device),
                                                               m.to(device))
    M, I, ref = oracle.fused_fwd_ref(H, W, b, m)
    A = oracle.logit_at(H.abs(), W.abs(), b.abs(), m.abs(), I)
    D = H.shape[-1]
    bound = (2.0 ** -18 * M + (D + 2) * 2.0 ** -24 * A) / (1 + M) + 2.0 ** -23 + 2.0 ** -21 * ref
    err = (r32.cpu().to(F64) - ref).abs()
    assert bool((err <= bound).all()), float((err - bound).max())
    say(f"  max |reps - log1p(M)| = {float(err.max()):.3e}, mean bound {float(bound.mean()):.3e}")


def test_bwd_accepts_reference_int64_index(device):
    """sparton::fused_sparton_bwd also takes the int64 indices the reference's ops exchange
    (sparton_kernel.py:658-667): same gradients as with int32; out-of-range values raise."""
    say("bwd with int64 max_idx")
    H, W, b, m, G = make_case("bf16", 3, 77, 64, 1000, True, "int64")
    Hd, Wd, bd, md, Gd = (t.to(device) for t in (H, W, b, m, G))
    reps, idx = torch.ops.sparton.fused_sparton_fwd(Hd, Wd, bd, md)
    a = torch.ops.sparton.fused_sparton_bwd(Gd, reps, idx, Hd, Wd, bd, md)
    c = torch.ops.sparton.fused_sparton_bwd(Gd, reps, idx.long(), Hd, Wd, bd, md)
    torch.cuda.synchronize()
    for x, y in zip(a, c):
        assert torch.equal(x, y)
    bad = idx.long().clone()
    bad[0, 0] = H.shape[1]
    with pytest.raises(ValueError, match="max_idx values"):
        torch.ops.sparton.fused_sparton_bwd(Gd, reps, bad, Hd, Wd, bd, md)



def test_autocast_weight_cast_is_cached_until_updated(device):
    """Under autocast over fp32 parameters the head casts W once and reuses the copy while W
    is unchanged (two calls per training step share it); an optimizer step, which updates W
    in place, makes the next call cast again, so its reps follow the new weights."""
    say("autocast cast cache and optimizer step")
    B, S, D, V = 3, 40, 64, 900
    g = torch.Generator().manual_seed(9)
    head = sparton.SpartonHead(V, D, use_bias=True).to(device)
    H = torch.randn(B, S, D, generator=g).to(device).requires_grad_()
    m = torch.ones(B, S, dtype=torch.long, device=device)
    opt = torch.optim.SGD(head.parameters(), lr=0.5)

    def run():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            return head(H, m)

    r1 = run()
    w1 = head._cast_cache._entries["weight"][1]
    r2 = run()
    assert head._cast_cache._entries["weight"][1] is w1   # reused, not cast again
    assert torch.equal(r1, r2)
    (r1.float().sum() + r2.float().sum()).backward()
    opt.step()
    opt.zero_grad(set_to_none=True)
    r3 = run()
    assert head._cast_cache._entries["weight"][1] is not w1
    ref = oracle.torch_head(H.detach().cpu().bfloat16().double(),
                            head.weight.detach().cpu().bfloat16().double(),
                            head.bias.detach().cpu().bfloat16().double(), m.cpu())
    torch.testing.assert_close(r3.detach().cpu().double(), ref, **FWD_TOL)
    assert not torch.equal(r3, r1)
    with torch.no_grad():   # inference under autocast uses the same copy
        with torch.autocast("cuda", dtype=torch.bfloat16):
            r4 = head(H, m)
    assert torch.equal(r4, r3.detach())

    def ref_now():
        return oracle.torch_head(H.detach().cpu().bfloat16().double(),
                                 head.weight.detach().cpu().bfloat16().double(),
                                 head.bias.detach().cpu().bfloat16().double(), m.cpu())

    # A write through .data is not versioned by torch; the backward dropped the copies, so
    # the next forward sees it (optimizers that update p.data after backward).
    r3.float().sum().backward()
    head.weight.data.mul_(-1.0)
    head.bias.data.add_(0.05)
    r5 = run()
    torch.testing.assert_close(r5.detach().cpu().double(), ref_now(), **FWD_TOL)
    assert not torch.equal(r5, r3)
    # A new parameter object (here likely at the freed address of the old one, version 0)
    # is a new key.
    r5.float().sum().backward()
    with torch.no_grad():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            head(H, m)   # caches a copy of the current weight for inference
    new_w = head.weight.detach().clone() * 2.0
    head.weight = None
    head.weight = torch.nn.Parameter(new_w)
    del new_w
    with torch.no_grad():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            r6 = head(H, m)
    torch.testing.assert_close(r6.cpu().double(), ref_now(), **FWD_TOL)


@pytest.mark.parametrize("use_bias", [True, False])
def test_eager_cpp_head_equals_custom_ops(use_bias, device):
    """SpartonHead's eager path (the C++ op sparton_eager::head_train, autograd in C++) gives
    bitwise the reps and gradients of the torch.library training op with its Python autograd,
    and inference (sparton_eager::head_encode) the reps of sparton::fused_sparton_encode."""
    from sparton_amd import _eager
    say(f"C++ eager head vs custom ops, bias={use_bias}")
    H, W, b, m, G = make_case("bf16", 4, 150, 128, 2000, use_bias, "int64", seed=4)
    Hd, Wd, md, Gd = H.to(device), W.to(device), m.to(device), G.to(device)
    bd = b.to(device) if b is not None else None
    outs = []
    for path in ("eager", "op"):
        h = Hd.clone().requires_grad_()
        w = Wd.clone().requires_grad_()
        bb = bd.clone().requires_grad_() if bd is not None else None
        if path == "eager":
            r = _eager.load().head_train(h, w, bb, md)
        else:
            r = torch.ops.sparton.fused_sparton_fwd_train(h, w, bb, md)[0]
        r.backward(Gd)
        outs.append([r.detach(), h.grad, w.grad] + ([bb.grad] if bb is not None else []))
    torch.cuda.synchronize()
    for a, c in zip(*outs):
        assert torch.equal(a, c)
    e = _eager.load().head_encode(Hd, Wd, bd, md)
    assert torch.equal(e, torch.ops.sparton.fused_sparton_encode(Hd, Wd, bd, md))
    head = sparton.SpartonHead(2000, 128, use_bias=use_bias).to(device).bfloat16()
    with torch.no_grad():
        head.weight.copy_(Wd)
        if use_bias:
            head.bias.copy_(bd)
    assert torch.equal(head(Hd, md), e)  # no grad needed: the module takes head_encode


def _sweep_cases(seed, n):
    import random
    rng = random.Random(seed)
    out = []
    for i in range(n):
        dt = rng.choice(["bf16", "fp16", "fp32"])
        B = rng.choice([1, 2, 3, 5, 8, 17])
        S = rng.choice([1, 7, 16, 31, 64, 100])
        D = rng.choice([8, 16, 64, 72, 200, 256]) if dt != "fp32" else rng.choice([4, 8, 64, 132, 256])
        V = rng.choice([1, 31, 256, 300, 1000])
        masks = ["int64", "bool", "holes", "frac", "int32"] + (["gaps"] if B >= 2 else [])
        prec = rng.choice(["highest", "high"]) if dt == "fp32" else "highest"
        out.append(((dt, B, S, D, V, rng.random() < 0.5, rng.choice(masks)), prec, i))
    return out


@pytest.mark.parametrize("case,prec,seed", _sweep_cases(7, 12),
                         ids=lambda x: "-".join(map(str, x)) if isinstance(x, tuple) else str(x))
def test_random_sweep(case, prec, seed, device):
    """Seeded random shapes, dtypes, masks and (fp32) matmul precisions through the training
    forward and the reference backward, against the oracle: edge sizes (V = 1, S = 1, D = 4,
    K tails, ragged batch rows) mixed as a user's calls would mix them."""
    say(f"sweep case {case} precision {prec}")
    prev = torch.get_float32_matmul_precision()
    try:
        torch.set_float32_matmul_precision(prec)
        H, W, b, m, G = make_case(*case, seed=seed)
        reps, idx, reps32, dH, dW, db = run_fwd_bwd(H, W, b, m, G, device)
    finally:
        torch.set_float32_matmul_precision(prev)
    n, bad = check_fwd(H, W, b, m, reps, idx, split=(prec == "high"))
    check_bwd_isolated(H, W, b, m, G, reps32, idx, dH, dW, db)
    say(f"  checked {n} entries, {bad} near-tie argmax differences")
