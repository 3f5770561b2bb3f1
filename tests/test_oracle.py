"""Pin the CPU oracle (oracle/sparton_ref.py) before trusting it as the checker.

Every oracle function is checked against something other than its own formula:
pure-Python loops, fp64 autograd of the torch head, closed-form known answers,
invariants, and the committed fixtures. The last tests plant plausible mistakes
in copies of the oracle and show that these checks catch them.
"""
import glob
import math
import os

import numpy as np
import pytest
import torch

import oracle
from sparton_amd.workloads import WORKLOADS, make_inputs

F64 = torch.float64
GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))


def rand_case(B, S, D, V, seed, bias=True, ties=False, mask="pad"):
    g = torch.Generator().manual_seed(seed)
    if ties:
        H = torch.randint(-1, 2, (B, S, D), generator=g).to(F64)
        W = torch.randint(-1, 2, (V, D), generator=g).to(F64)
    else:
        H = torch.randn(B, S, D, generator=g, dtype=F64)
        W = torch.randn(V, D, generator=g, dtype=F64) * 0.3
    b = (torch.randn(V, generator=g, dtype=F64) * 0.2) if bias else None
    if mask == "pad":
        lens = torch.randint(1, S + 1, (B,), generator=g)
        m = (torch.arange(S)[None] < lens[:, None]).long()
    else:
        m = (torch.rand(B, S, generator=g) < 0.5).long()
    G = torch.rand(B, V, generator=g, dtype=F64)
    return H, W, b, m, G


# ---- forward -------------------------------------------------------------------

@pytest.mark.parametrize("seed,ties,bias,mask", [(0, False, True, "pad"), (1, True, True, "pad"),
                                                 (2, True, False, "holes"), (3, False, False, "holes")])
def test_fwd_matches_brute_force(seed, ties, bias, mask):
    H, W, b, m, _ = rand_case(2, 7, 5, 9, seed, bias=bias, ties=ties, mask=mask)
    M, I, reps = oracle.fused_fwd_ref(H, W, b, m)
    bM, bI, brep = oracle.brute_fwd(H, W, b, m)
    assert torch.allclose(M, torch.tensor(bM, dtype=F64), rtol=1e-13, atol=1e-13)
    assert torch.equal(I, torch.tensor(bI))
    assert torch.allclose(reps, torch.tensor(brep, dtype=F64), rtol=1e-13, atol=1e-13)


def test_fwd_equals_torch_head_values():
    H, W, b, m, _ = rand_case(3, 11, 6, 20, 5)
    _, _, reps = oracle.fused_fwd_ref(H, W, b, m)
    assert torch.allclose(reps, oracle.torch_head(H, W, b, m), rtol=1e-13, atol=1e-13)


def test_fwd_ties_pick_lowest_s_like_torch_max():
    # torch.max(dim) returns the first maximal index; the oracle must agree where M > 0.
    H, W, b, m, _ = rand_case(2, 9, 4, 30, 7, ties=True)
    M, I, _ = oracle.fused_fwd_ref(H, W, b, m)
    x = (H @ W.T + b) * m.unsqueeze(-1)
    first = x.max(dim=1).indices
    pos = M > 0
    assert int(((x == M.unsqueeze(1)).sum(1) > 1)[pos].sum()) > 0, "case has no ties"
    assert torch.equal(I[pos], first[pos])
    assert torch.equal(I[~pos], torch.zeros_like(I[~pos]))


def test_kat_zero_weight_constant_bias():
    B, S, D, V, c = 3, 6, 8, 5, 0.7
    H = torch.randn(B, S, D, dtype=F64)
    W = torch.zeros(V, D, dtype=F64)
    b = torch.full((V,), c, dtype=F64)
    m = torch.tensor([[1, 1, 1, 0, 0, 0], [0, 0, 1, 1, 0, 0], [0, 0, 0, 0, 0, 1]])
    M, I, reps = oracle.fused_fwd_ref(H, W, b, m)
    assert torch.allclose(reps, torch.full((B, V), math.log1p(c), dtype=F64))
    assert I.tolist() == [[0] * V, [2] * V, [5] * V]   # first valid position wins the tie


def test_kat_all_masked_row_and_negative_logits():
    H, W, b, m, _ = rand_case(2, 5, 4, 6, 9)
    m[0] = 0
    b = torch.full((6,), -100.0, dtype=F64)            # every logit negative in row 1
    M, I, reps = oracle.fused_fwd_ref(H, W, b, m)
    assert torch.all(reps == 0) and torch.all(I == 0)


def test_kat_single_position_is_elementwise():
    H, W, b, m, _ = rand_case(4, 1, 6, 7, 10)
    m[:] = 1
    _, I, reps = oracle.fused_fwd_ref(H, W, b, m)
    expect = torch.log1p(torch.relu(torch.nn.functional.linear(H[:, 0], W, b)))
    assert torch.allclose(reps, expect) and torch.all(I == 0)


def test_kat_one_hot_identity():
    # H rows one-hot times a value, W = identity: x[b,s,v] = value if hot index == v.
    B, S, V = 2, 4, 4
    H = torch.zeros(B, S, V, dtype=F64)
    vals = torch.tensor([[0.5, 2.0, 1.0, 3.0], [1.5, 0.25, 4.0, 0.75]], dtype=F64)
    hot = torch.tensor([[0, 1, 1, 3], [2, 2, 0, 1]])
    for bb in range(B):
        for s in range(S):
            H[bb, s, hot[bb, s]] = vals[bb, s]
    m = torch.ones(B, S, dtype=torch.long)
    M, I, reps = oracle.fused_fwd_ref(H, torch.eye(V, dtype=F64), None, m)
    # row 0: v0 <- s0 (0.5); v1 <- s1 (2.0 beats s2's 1.0); v2 never hot; v3 <- s3 (3.0)
    # row 1: v0 <- s2 (4.0); v1 <- s3 (0.75); v2 <- s0 (1.5 beats s1's 0.25); v3 never hot
    assert M.tolist() == [[0.5, 2.0, 0.0, 3.0], [4.0, 0.75, 1.5, 0.0]]
    assert I.tolist() == [[0, 1, 0, 3], [2, 3, 0, 0]]


def test_invariants_permutation_chunking_padding():
    H, W, b, m, _ = rand_case(3, 8, 5, 17, 11)
    M, I, reps = oracle.fused_fwd_ref(H, W, b, m)
    perm = torch.randperm(17, generator=torch.Generator().manual_seed(0))
    Mp, Ip, _ = oracle.fused_fwd_ref(H, W[perm], b[perm], m)
    assert torch.equal(Mp, M[:, perm]) and torch.equal(Ip, I[:, perm])
    Mc, Ic, _ = oracle.fused_fwd_ref(H, W, b, m, v_chunk=5)
    assert torch.equal(Mc, M) and torch.equal(Ic, I)
    H2 = torch.cat([H, torch.randn(3, 4, 5, dtype=F64)], 1)
    m2 = torch.cat([m, torch.zeros(3, 4, dtype=torch.long)], 1)
    M2, I2, _ = oracle.fused_fwd_ref(H2, W, b, m2)
    assert torch.equal(M2, M) and torch.equal(I2, I)
    assert torch.all(reps >= 0) and torch.all(I < 8)
    Bi = torch.arange(3).view(3, 1)
    assert torch.all(m[Bi, I][M > 0] == 1)


def test_torch_head_chunked_identical():
    H, W, b, m, _ = rand_case(2, 6, 4, 23, 12)
    assert torch.equal(oracle.torch_head_chunked(H, W, b, m, v_chunk=7), oracle.torch_head(H, W, b, m))


def test_logit_at_matches_dense():
    H, W, b, m, _ = rand_case(2, 6, 4, 13, 13)
    idx = torch.randint(0, 6, (2, 13))
    x = (H @ W.T + b) * m.unsqueeze(-1)
    assert torch.allclose(oracle.logit_at(H, W, b, m, idx, v_chunk=5), x.gather(1, idx.unsqueeze(1)).squeeze(1))


# ---- backward ------------------------------------------------------------------

def test_torch_head_gradcheck_fp64():
    H, W, b, m, _ = rand_case(2, 4, 3, 5, 14)
    H.requires_grad_(); W.requires_grad_(); b.requires_grad_()
    assert torch.autograd.gradcheck(lambda h, w, bb: oracle.torch_head(h, w, bb, m), (H, W, b))


@pytest.mark.parametrize("bias,mask", [(True, "pad"), (False, "holes")])
def test_sparse_bwd_equals_torch_head_autograd(bias, mask):
    H, W, b, m, G = rand_case(3, 8, 6, 19, 15, bias=bias, mask=mask)
    G[G < 0.3] = 0                                       # sparse upstream grad
    Hr, Wr = H.clone().requires_grad_(), W.clone().requires_grad_()
    br = b.clone().requires_grad_() if bias else None
    oracle.torch_head(Hr, Wr, br, m).backward(G)
    _, I, reps = oracle.fused_fwd_ref(H, W, b, m)
    dH, dW, db = oracle.fused_bwd_ref(G, reps, I, H, W, bias, m)
    assert torch.allclose(dH, Hr.grad, rtol=1e-12, atol=1e-12)
    assert torch.allclose(dW, Wr.grad, rtol=1e-12, atol=1e-12)
    if bias:
        assert torch.allclose(db, br.grad, rtol=1e-12, atol=1e-12)
    else:
        assert db is None


def test_sparse_bwd_fractional_mask_matches_autograd():
    H, W, b, m, G = rand_case(2, 6, 4, 11, 16)
    mf = torch.tensor([[1.0, 0.5, 0.25, 1.0, 0.0, 0.75], [0.5, 0.5, 0.0, 1.0, 1.0, 0.25]], dtype=F64)
    Hr, Wr, br = H.clone().requires_grad_(), W.clone().requires_grad_(), b.clone().requires_grad_()
    oracle.torch_head(Hr, Wr, br, mf).backward(G)
    _, I, reps = oracle.fused_fwd_ref(H, W, b, mf)
    dH, dW, db = oracle.fused_bwd_ref(G, reps, I, H, W, True, mf)
    assert torch.allclose(dH, Hr.grad) and torch.allclose(dW, Wr.grad) and torch.allclose(db, br.grad)


def test_sparse_bwd_matches_brute_force():
    H, W, b, m, G = rand_case(2, 5, 4, 7, 17, ties=True)
    _, I, reps = oracle.fused_fwd_ref(H, W, b, m)
    dH, dW, db = oracle.fused_bwd_ref(G, reps, I, H, W, True, m)
    bH, bW, bb = oracle.brute_bwd(G, reps, I, H, W, True, m)
    assert torch.allclose(dH, torch.tensor(bH, dtype=F64))
    assert torch.allclose(dW, torch.tensor(bW, dtype=F64))
    assert torch.allclose(db, torch.tensor(bb, dtype=F64))


def test_sparse_bwd_invariants():
    H, W, b, m, G = rand_case(4, 9, 6, 25, 18)
    _, I, reps = oracle.fused_fwd_ref(H, W, b, m)
    dH, dW, db = oracle.fused_bwd_ref(G, reps, I, H, W, True, m, chunk=7)
    gp = oracle.grad_coeff(G, reps, I, m)
    assert torch.allclose(db, gp.sum(0))
    assert torch.allclose(dH.sum(1), gp @ W)                       # sum_s dH = G' W
    Hg = H[torch.arange(4).view(4, 1), I]                         # [B,V,D] gathered rows
    assert torch.allclose(dW, torch.einsum("bv,bvd->vd", gp, Hg))
    onehot = torch.nn.functional.one_hot(I, 9).to(F64)            # dH = (G' one-hot)^T W per b
    assert torch.allclose(dH, torch.einsum("bv,bvs,vd->bsd", gp, onehot, W))


# ---- fixtures -------------------------------------------------------------------

@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p) for p in GOLDEN])
def test_oracle_reproduces_golden_fixture(path):
    z = np.load(path)
    t = {k: torch.from_numpy(z[k]) for k in z.files}
    bias = t.get("bias")
    M, I, reps = oracle.fused_fwd_ref(t["hidden"], t["weight"], bias, t["mask"])
    assert torch.equal(I, t["I"]) and torch.allclose(M, t["M"], rtol=0, atol=0)
    dH, dW, db = oracle.fused_bwd_ref(t["grad"], t["reps"], t["I"], t["hidden"], t["weight"],
                                      bias is not None, t["mask"])
    assert torch.allclose(dH, t["dH"], rtol=1e-12, atol=1e-12)
    assert torch.allclose(dW, t["dW"], rtol=1e-12, atol=1e-12)
    if bias is not None:
        assert torch.allclose(db, t["dbias"], rtol=1e-12, atol=1e-12)


def test_fixtures_present_and_have_ties():
    assert len(GOLDEN) >= 5
    z = np.load([p for p in GOLDEN if "ties" in p][0])
    H, W, b, m = (torch.from_numpy(z[k]) for k in ("hidden", "weight", "bias", "mask"))
    x = (H @ W.T + b) * m.unsqueeze(-1)
    M = torch.from_numpy(z["M"])
    assert int((((x == M.unsqueeze(1)).sum(1) > 1) & (M > 0)).sum()) > 0


# ---- planted mistakes: each mutated oracle must fail one of the checks above -----

def _wrong_tie(H, W, b, m):  # highest s wins ties
    M, I, r = oracle.fused_fwd_ref(H, W, b, m)
    x = (H @ W.T + (0 if b is None else b)) * m.unsqueeze(-1)
    S = H.shape[1]
    last = torch.where(x == M.unsqueeze(1), torch.arange(S).view(1, S, 1), -1).max(1).values
    return M, torch.where(M > 0, last, 0), r


def _dropped_bias(H, W, b, m):
    return oracle.fused_fwd_ref(H, W, None, m)


def _mask_before_bias(H, W, b, m):  # x = H.W*m + b instead of (H.W + b)*m
    x = (H @ W.T) * m.unsqueeze(-1) + b
    M = x.max(1).values.clamp(min=0)
    return M, x.max(1).indices * (M > 0), torch.log1p(M)


@pytest.mark.parametrize("mutant", [_wrong_tie, _dropped_bias, _mask_before_bias])
def test_planted_forward_mistakes_are_caught(mutant):
    H, W, b, m, _ = rand_case(2, 7, 5, 9, 1, ties=True)
    M, I, _ = mutant(H, W, b, m)
    bM, bI, _ = oracle.brute_fwd(H, W, b, m)
    caught = not (torch.allclose(M, torch.tensor(bM, dtype=F64)) and torch.equal(I, torch.tensor(bI)))
    assert caught


def test_planted_backward_mistake_is_caught():
    # g' without the exp(-reps) factor must disagree with fp64 autograd of the torch head.
    H, W, b, m, G = rand_case(2, 6, 4, 9, 3)
    Wr = W.clone().requires_grad_()
    oracle.torch_head(H, Wr, b, m).backward(G)
    _, I, reps = oracle.fused_fwd_ref(H, W, b, m)
    _, dW_bad, _ = oracle.fused_bwd_ref(G, torch.zeros_like(reps) + 1e-300 * (reps > 0), I, H, W, True, m)
    assert not torch.allclose(dW_bad, Wr.grad)


# ---- workloads --------------------------------------------------------------------

def test_workload_generator_is_seeded_and_shaped():
    w = WORKLOADS[2].scaled(B=4, S=20, D=16, V=50)
    a, b2 = make_inputs(w), make_inputs(w)
    assert torch.equal(a.hidden, b2.hidden) and torch.equal(a.grad, b2.grad)
    assert a.hidden.dtype == torch.bfloat16 and a.mask.dtype == torch.int64
    assert a.mask.shape == (4, 20) and torch.equal(a.mask.sum(1), a.lengths)
    assert WORKLOADS[5].bias is None and WORKLOADS[3].full_rows == 4
