"""CPU checks of the drop-in boundary: the C-ABI library, the Python ops and the
SpartonHead module surface. Nothing here launches a kernel."""
import ctypes
import os
import re
import subprocess
import sys

import pytest
import torch

import sparton
import sparton_amd
from sparton_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sparton.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sparton_[a-z_]+)\s*\(", text)))


def test_library_is_built_and_exports_every_declared_symbol():
    L = _lib.load()
    declared = header_functions()
    assert set(declared) == set(_lib.EXPORTED_SYMBOLS)
    for name in declared:
        assert hasattr(L, name), name
    nm = subprocess.run(["nm", "-D", "--defined-only", _lib.lib_path()], capture_output=True, text=True)
    exported = {ln.split()[-1] for ln in nm.stdout.splitlines() if " T " in ln}
    assert exported == set(declared), exported ^ set(declared)


def test_host_side_entry_points():
    L = _lib.load()
    assert L.sparton_abi_version() == _lib.ABI_VERSION
    assert L.sparton_strerror(0) == b"success"
    for code in (-1, -2, -3, -4, -5, 7, -99):
        assert len(L.sparton_strerror(code)) > 0
    max_s, max_b = _lib.limits()
    assert max_s == max_b == 2**31 - 1
    ws = L.sparton_bwd_workspace_bytes(32, 256, 768, 30522)
    assert ws % 256 == 0 and ws >= 32 * 30522 * 8 + 2 * 32 * 256 * 4
    assert L.sparton_bwd_workspace_bytes(0, 256, 768, 30522) == 0
    fws = L.sparton_fwd_workspace_bytes(32, 256, 768, 30522, 1)
    # plan (flags, counts, block list) + two partial rows of V (max, argmax) per row tile
    assert fws % 256 == 0 and fws >= 32 * 2 * 30522 * 8
    assert L.sparton_fwd_workspace_bytes(0, 256, 768, 30522, 1) == 0


# Argument checks that return before any HIP call (fake, never-dereferenced pointers).
P = 0x10000  # 16-byte aligned dummy address


def fwd(**kw):
    a = dict(hidden=P, weight=P, bias=None, mask=P, mask_dtype=0, reps=P, argmax=P, reps32=None,
             B=2, S=4, D=64, V=10, dtype=1, ws=P, ws_bytes=1 << 30, stream=None)
    a.update(kw)
    return _lib.load().sparton_fwd(*a.values())


def bwd(**kw):
    a = dict(grad=P, reps=P, reps_dtype=1, argmax=P, mask=P, mask_dtype=0, hidden=P, weight=P,
             dH=P, dW=P, db=None, grad_dtype=0, ws=None, ws_bytes=0, B=2, S=4, D=64, V=10, dtype=1,
             stream=None)
    a.update(kw)
    return _lib.load().sparton_bwd(*a.values())


@pytest.mark.parametrize("kw,code", [
    (dict(B=-1), -1), (dict(dtype=3), -1), (dict(mask_dtype=6), -1), (dict(hidden=None), -1),
    (dict(D=60), -1), (dict(D=4, dtype=1), -1), (dict(hidden=P + 8), -2), (dict(weight=P + 4), -2),
    (dict(B=0), 0), (dict(V=0), 0), (dict(ws=None), -4), (dict(ws_bytes=16), -4),
    (dict(ws=P + 16), -2),
    (dict(S=1 << 24), -3),                # a batch row of H reaches 2^31 bytes
    (dict(S=20000, ws_bytes=16), -4),     # S > 16384 is accepted (stops at the workspace)
    (dict(dtype=1 | 0x100), -1),          # SPARTON_F32_SPLIT only with SPARTON_F32
    (dict(dtype=0x200), -1),              # no other flag bits
    (dict(dtype=0x100, D=62), -1),        # fp32 rows of 248 bytes: not a multiple of 16
    (dict(dtype=0x100, ws=None), -4),     # fp32 split is accepted (stops at the workspace)
    (dict(dtype=0x100, B=0), 0),
])
def test_fwd_argument_validation(kw, code):
    assert fwd(**kw) == code


def test_fwd_dtype_code_follows_torch_fp32_precision():
    """fp32 takes the bf16 hi/lo split (SPARTON_F32_SPLIT) under torch's 'high' or 'medium'
    float32 matmul precision (the reference sets 'high' at import, sparton_kernel.py:14),
    exact fp32 under 'highest'; 16-bit dtypes never carry the flag."""
    prev = torch.get_float32_matmul_precision()
    try:
        for prec, want in (("highest", 0), ("high", 0x100), ("medium", 0x100)):
            torch.set_float32_matmul_precision(prec)
            assert _lib.fwd_dtype_code(torch.float32) == want
            assert _lib.fwd_dtype_code(torch.bfloat16) == 1
            assert _lib.fwd_dtype_code(torch.float16) == 2
    finally:
        torch.set_float32_matmul_precision(prev)


@pytest.mark.parametrize("kw,code", [
    (dict(S=-2), -1), (dict(dtype=-1), -1), (dict(reps_dtype=3), -1), (dict(grad_dtype=2), -1),
    (dict(reps_dtype=2), -1),  # reps must be fp32 or the parameters' dtype (bf16 here)
    (dict(dtype=0x100), -1),   # the split flag is the forward's only
    (dict(grad=None), -1), (dict(dH=P + 4, grad_dtype=1, ws=P, ws_bytes=1 << 30), -2),
    (dict(dW=P + 8, grad_dtype=0, ws=P, ws_bytes=1 << 30), -2),
    (dict(weight=None), -1),
    (dict(D=12), -1), (dict(dH=P + 4), -2), (dict(ws=None), -4), (dict(ws=P, ws_bytes=16), -4),
    (dict(S=1 << 30), -3), (dict(B=1 << 28), -3),   # B * S or B * V reaches 2^31
    (dict(S=20000), -4), (dict(B=9000), -4),         # accepted (dH passes over windows / chunks)
    (dict(dH=None, dW=None, db=None), 0),
])
def test_bwd_argument_validation(kw, code):
    assert bwd(**kw) == code


def test_fwd_profile_requires_time_output():
    a = dict(hidden=P, weight=P, bias=None, mask=P, mask_dtype=0, reps=P, argmax=P, reps_f32=None,
             B=2, S=4, D=64, V=10, dtype=1, ws=P, ws_bytes=1 << 30, stream=None, main_ms=None)
    assert _lib.load().sparton_fwd_profile(*a.values()) == -1


def test_strerror_from_python_check():
    with pytest.raises(RuntimeError, match="invalid argument"):
        _lib.check(-1, "x")


def test_missing_library_fails_loudly():
    code = ("import os, torch, sparton_amd.ops as o\n"
            "h=torch.zeros(1,1,8,dtype=torch.bfloat16,device='meta')\n"
            "from sparton_amd import _lib\n"
            "try:\n    _lib.load()\nexcept RuntimeError as e:\n    print('RAISED', e)\n")
    env = dict(os.environ, SPARTON_HIP_LIB="/nonexistent/libsparton_hip.so", PYTHONPATH=ROOT)
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, cwd=ROOT)
    assert "RAISED" in out.stdout and "python -m sparton_amd.build" in out.stdout, out.stderr


def test_product_never_imports_oracle():
    pkg = os.path.join(ROOT, "sparton_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith(".py"):
                src = open(os.path.join(dirpath, f)).read()
                assert not re.search(r"^\s*(from|import)\s+oracle", src, re.M), f


# ---- Python ops and module (CPU / meta tensors only) ----------------------------------

def test_ops_reject_cpu_tensors_like_reference_assert():
    H = torch.zeros(2, 4, 8)
    W = torch.zeros(10, 8)
    m = torch.ones(2, 4, dtype=torch.long)
    with pytest.raises(RuntimeError, match="only supports ROCm/HIP device"):
        torch.ops.sparton.fused_sparton_fwd(H, W, None, m)
    with pytest.raises(RuntimeError, match="only supports ROCm/HIP device"):
        torch.ops.sparton.fused_sparton_encode(H, W, None, m)


@pytest.mark.parametrize("bad", ["hidden_rank", "dim", "bias", "mask", "dtype", "D"])
def test_ops_validate_shapes(bad):
    from sparton_amd.ops import _validate
    H, W, b, m = torch.zeros(2, 4, 16), torch.zeros(10, 16), torch.zeros(10), torch.ones(2, 4)
    if bad == "hidden_rank":
        H = H[0]
    elif bad == "dim":
        W = torch.zeros(10, 8)
    elif bad == "bias":
        b = torch.zeros(9)
    elif bad == "mask":
        m = torch.ones(2, 5)
    elif bad == "dtype":
        W = W.double()
    elif bad == "D":
        H, W = torch.zeros(2, 4, 6), torch.zeros(10, 6)
    with pytest.raises((ValueError, TypeError)):
        _validate(H, W, b, m, "op")


def test_fake_kernels_give_reference_metadata():
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        H = torch.empty(3, 5, 16, dtype=torch.bfloat16)
        W = torch.empty(40, 16, dtype=torch.bfloat16)
        b = torch.empty(40, dtype=torch.bfloat16)
        m = torch.empty(3, 5, dtype=torch.long)
        r, i = torch.ops.sparton.fused_sparton_fwd(H, W, b, m)
        assert r.shape == (3, 40) and r.dtype == torch.bfloat16 and i.dtype == torch.int32
        e = torch.ops.sparton.fused_sparton_encode(H, W, None, m)
        assert e.shape == (3, 40)
        r3, i3, r32 = torch.ops.sparton.fused_sparton_fwd_train(H, W, b, m)
        assert r3.dtype == torch.bfloat16 and i3.dtype == torch.int32 and r32.dtype == torch.float32
        dh, dw, db = torch.ops.sparton.fused_sparton_bwd(r, r32, i, H, W, b, m)
        assert dh.shape == H.shape and dw.shape == W.shape and db.shape == (40,)
        assert dh.dtype == dw.dtype == db.dtype == torch.float32
        th, tw, tb = torch.ops.sparton.fused_sparton_bwd_train(r, r32, i, H, W, b, m)
        assert th.dtype == tw.dtype == tb.dtype == torch.bfloat16 and tw.shape == W.shape
        _, _, db0 = torch.ops.sparton.fused_sparton_bwd(r, r, i, H, W, None, m)
        assert db0.shape == (0,)


def test_module_surface_matches_reference():
    assert sparton.SpartonHead is sparton_amd.SpartonHead
    h = sparton.SpartonHead(50, 16, use_bias=True)
    assert h.weight.shape == (50, 16) and h.bias.shape == (50,)
    assert sorted(dict(h.named_parameters())) == ["bias", "weight"]
    bound = 1 / 16 ** 0.5
    assert h.bias.abs().max() <= bound and h.weight.abs().max() <= bound  # kaiming_uniform(a=sqrt 5)
    h2 = sparton.SpartonHead(50, 16)
    assert h2.bias is None and list(dict(h2.named_parameters())) == ["weight"]


def test_tie_weights_aliases_decoder_and_load_copies():
    dec = torch.nn.Linear(16, 50)
    h = sparton.SpartonHead(dec.out_features, dec.in_features, use_bias=True)
    h.tie_weights(dec)
    assert h.weight is dec.weight and h.bias is dec.bias
    h3 = sparton.SpartonHead(50, 16, use_bias=True)
    w, b = torch.randn(50, 16), torch.randn(50)
    h3.load({"weight": w, "bias": b})
    assert torch.equal(h3.weight.data, w) and torch.equal(h3.bias.data, b)


def test_c_header_compiles_as_c():
    src = os.path.join(ROOT, "include", "sparton.h")
    out = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-fsyntax-only", "-x", "c", src],
                         capture_output=True, text=True)
    assert out.returncode == 0, out.stderr


# ---- the MLM transform entry points (argument checks only; nothing is launched) ----
def xf_fwd(**kw):
    a = dict(z=P, bd=P, g=P, bt=P, eps=1e-12, y=P, mean=P, rstd=P, M=8, D=64, dtype=1, stream=None)
    a.update(kw)
    return _lib.load().sparton_transform_fwd(*a.values())


def xf_bwd(**kw):
    a = dict(dy=P, z=P, bd=P, g=P, mean=P, rstd=P, dz=P, dg=None, dbt=None, dbd=None, ws=P,
             ws_bytes=1 << 30, M=8, D=64, dtype=1, stream=None)
    a.update(kw)
    return _lib.load().sparton_transform_bwd(*a.values())


@pytest.mark.parametrize("kw,code", [
    (dict(M=-1), -1), (dict(dtype=3), -1), (dict(D=62), -1), (dict(z=None), -1),
    (dict(eps=-1.0), -1), (dict(eps=float("nan")), -1), (dict(bd=P + 4), -2), (dict(D=3076), -3),
    (dict(M=0), 0), (dict(D=0), 0),
])
def test_transform_fwd_argument_validation(kw, code):
    assert xf_fwd(**kw) == code


@pytest.mark.parametrize("kw,code", [
    (dict(M=-1), -1), (dict(D=6), -1), (dict(dy=None), -1), (dict(ws=None), -4),
    (dict(ws_bytes=16), -4), (dict(ws=P + 4), -2), (dict(g=P + 8), -2), (dict(D=4096), -3),
    (dict(M=0), 0),
])
def test_transform_bwd_argument_validation(kw, code):
    assert xf_bwd(**kw) == code


def test_transform_workspace_size():
    L = _lib.load()
    # fp32 column partials of (dy * xhat, dy, dz) per backward workgroup: 8 waves (4 when
    # D > 1024) of R rows each, R = ceil(M / (waves * 256)) clamped to [1, 32]
    part = lambda blocks, D: blocks * 3 * D * 4
    assert L.sparton_transform_workspace_bytes(8192, 768) == part(256, 768)      # R = 4
    assert L.sparton_transform_workspace_bytes(33, 8) == part(5, 8)              # R = 1
    assert L.sparton_transform_workspace_bytes(65536, 768) == part(256, 768)     # R = 32
    assert L.sparton_transform_workspace_bytes(200000, 768) == part(782, 768)    # R capped
    assert L.sparton_transform_workspace_bytes(8192, 2048) == part(256, 2048)    # 4 waves, R = 8
    assert L.sparton_transform_workspace_bytes(0, 768) == 0


def test_transform_module_surface():
    dense, ln = torch.nn.Linear(64, 64), torch.nn.LayerNorm(64, eps=1e-12)
    m = sparton_amd.SpartonMLMTransform(dense, ln)
    assert m.dense.weight is dense.weight and m.layer_norm.weight is ln.weight  # shared, not copied

    class BertLike(torch.nn.Module):  # BertPredictionHeadTransform's attribute names
        def __init__(self):
            super().__init__()
            self.dense, self.LayerNorm = torch.nn.Linear(64, 64), torch.nn.LayerNorm(64)

    b = BertLike()
    assert sparton_amd.SpartonMLMTransform.from_hf(b).layer_norm is b.LayerNorm
    with pytest.raises(ValueError):
        sparton_amd.SpartonMLMTransform(torch.nn.Linear(64, 32), ln)
    # BERT's own transform module: erf gelu accepted, other activations refused
    from transformers import BertConfig
    from transformers.models.bert.modeling_bert import BertPredictionHeadTransform
    for act, ok in (("gelu", True), ("gelu_python", True), ("gelu_new", False), ("relu", False)):
        t = BertPredictionHeadTransform(BertConfig(hidden_size=64, hidden_act=act))
        if ok:
            assert sparton_amd.SpartonMLMTransform.from_hf(t).dense is t.dense
        else:
            with pytest.raises(ValueError, match="erf"):
                sparton_amd.SpartonMLMTransform.from_hf(t)
    with pytest.raises(RuntimeError, match="ROCm/HIP device tensors"):
        m(torch.randn(2, 3, 64))


# ---- the SPLADE loss entry points (argument checks only; nothing is launched) ----
def loss_fwd(**kw):
    a = dict(q=P, d=P, Bq=4, Bd=8, V=100, T=1.0, w_ce=1.0, w_l1=0.0, w_fl=0.0, out=P, probs=P,
             ws=P, ws_bytes=1 << 30, dtype=1, stream=None)
    a.update(kw)
    return _lib.load().sparton_loss_fwd(*a.values())


def loss_bwd(**kw):
    a = dict(q=P, d=P, probs=P, g=P, Bq=4, Bd=8, V=100, w_ce=1.0, w_l1=0.0, w_fl=0.0, gq=P, gd=P,
             dtype=1, stream=None)
    a.update(kw)
    return _lib.load().sparton_loss_bwd(*a.values())


@pytest.mark.parametrize("kw,code", [
    (dict(Bq=0), -1), (dict(V=0), -1), (dict(dtype=3), -1), (dict(Bq=9), -1),   # Bq > Bd
    (dict(q=None), -1), (dict(d=None), -1), (dict(probs=None), -1), (dict(out=None), -1),
    (dict(T=0.0), -1), (dict(T=float("inf")), -1), (dict(T=float("nan")), -1),
    (dict(Bq=1 << 28, Bd=1 << 28), -3), (dict(V=1 << 31), -3),
    (dict(ws=None), -4), (dict(ws_bytes=64), -4), (dict(ws=P + 4), -2),
])
def test_loss_fwd_argument_validation(kw, code):
    assert loss_fwd(**kw) == code


@pytest.mark.parametrize("kw,code", [
    (dict(Bq=0), -1), (dict(g=None), -1), (dict(gq=None), -1), (dict(gd=None), -1),
    (dict(probs=None), -1), (dict(Bq=9), -1), (dict(Bd=1 << 28), -3), (dict(V=1 << 31), -3),
    (dict(dtype=-1), -1),
])
def test_loss_bwd_argument_validation(kw, code):
    assert loss_bwd(**kw) == code


def loss_bwd_terms(**kw):
    import ctypes
    terms = (ctypes.c_void_p * 6)(P, None, None, None, None, None)
    a = dict(q=P, d=P, probs=P, terms=terms, Bq=4, Bd=8, V=100, w_ce=1.0, w_l1=0.0, w_fl=0.0, gq=P,
             gd=P, dtype=1, stream=None)
    a.update(kw)
    return _lib.load().sparton_loss_bwd_terms(*a.values())


@pytest.mark.parametrize("kw,code", [
    (dict(terms=None), -1), (dict(Bq=0), -1), (dict(gq=None), -1), (dict(gd=None), -1),
    (dict(probs=None), -1), (dict(Bq=9), -1), (dict(Bd=1 << 28), -3), (dict(V=1 << 31), -3),
    (dict(dtype=-1), -1),
])
def test_loss_bwd_terms_argument_validation(kw, code):
    assert loss_bwd_terms(**kw) == code


def test_loss_workspace_size():
    L = _lib.load()
    # fp32 partials per 64-column slice plus their sums: Bq*Bd scores, Bq + Bd row sums of
    # |x| and two sums of squared column sums
    assert L.sparton_loss_workspace_bytes(32, 32, 30522) == (477 + 1) * (1024 + 64 + 2) * 4
    assert L.sparton_loss_workspace_bytes(4, 0, 64) == 2 * (4 + 2) * 4
    assert L.sparton_loss_workspace_bytes(0, 4, 64) == 0
    # past 64 rows: 16 score tiles of 128 x 128 -> 32 vocabulary chunks of 960 columns, one
    # partial S each, S itself, per-slice row/column statistics plus their sums, and Bq row
    # CE terms
    assert L.sparton_loss_workspace_bytes(512, 512, 30522) == (
        32 * 512 * 512 + 512 * 512 + (477 + 1) * (512 + 512 + 2) + 512) * 4
    assert L.sparton_loss_workspace_bytes(300, 0, 1000) == ((16 + 1) * (300 + 2) + 300) * 4


def test_loss_module_surface():
    from sparton_amd import loss
    assert loss.get_reg_weight(50, 100, 1e-3) == pytest.approx(5e-4)
    assert loss.get_reg_weight(5, 0, 1e-3) == 1e-3
    with pytest.raises(RuntimeError, match="ROCm/HIP device tensors"):
        loss.splade_loss(torch.rand(2, 10), torch.rand(2, 10))
    assert callable(torch.ops.sparton.splade_loss_fwd) and callable(torch.ops.sparton.splade_loss_bwd)


def test_transform_dw_chunk_argument_validation():
    L = _lib.load()
    chunks = lambda **kw: L.sparton_transform_dz_chunks(*{**dict(dz=P, dzt=P, M=8192, D=768, C=8, dtype=1, stream=None), **kw}.values())
    csum = lambda **kw: L.sparton_transform_chunk_sum(*{**dict(part=P, out=P, C=8, n=768 * 768, dtype=1, stream=None), **kw}.values())
    assert chunks(M=8000) == -1          # M % C != 0
    assert chunks(M=8 * 96) == -1        # M / C not a multiple of 64
    assert chunks(C=0) == -1 and chunks(dtype=5) == -1 and chunks(dz=None) == -1
    assert chunks(dtype=0) == -1         # 16-bit types only
    assert chunks(D=740) == -1           # D % 64 != 0
    assert chunks(dz=P + 8) == -2
    assert chunks(M=0) == 0
    assert csum(n=6) == -1 and csum(C=0) == -1 and csum(out=None) == -1
    assert csum(part=P + 4) == -2
    assert csum(n=0) == 0


def test_transform_weight_grad_chunk_rule():
    """dW = dz^T x runs as a batched GEMM over C row chunks only for 16-bit types, M >= 2048,
    D % 64 == 0 and M % (64 C) == 0; C = 4 / 8 / 16 for M <= 4096 / <= 16384 / larger."""
    from sparton_amd.transform import _wgrad_chunks
    bf, f32 = torch.bfloat16, torch.float32
    assert _wgrad_chunks(8192, 768, bf) == 8
    assert _wgrad_chunks(4096, 768, torch.float16) == 4
    assert _wgrad_chunks(32768, 1024, bf) == 16
    assert _wgrad_chunks(8192, 768, f32) == 0          # fp32: one plain GEMM
    assert _wgrad_chunks(1024, 768, bf) == 0           # few rows
    assert _wgrad_chunks(8192, 740, bf) == 0           # D % 64 != 0
    assert _wgrad_chunks(8192 + 64, 768, bf) == 0      # M % (64 * 8) != 0


def test_fwd_noalloc_rejections_before_any_hip_call():
    """sparton_fwd_noalloc validates its arguments and its scratch limit before touching
    the device (fake, never-dereferenced pointers)."""
    L = _lib.load()
    cap = L.sparton_fwd_noalloc_max_workspace()
    assert cap == 32 << 20

    def call(**kw):
        a = dict(hidden=P, weight=P, bias=None, mask=P, mask_dtype=0, reps=P, argmax=P, reps32=None,
                 B=2, S=4, D=64, V=10, dtype=1, stream=None)
        a.update(kw)
        return L.sparton_fwd_noalloc(*a.values())

    assert call(B=-1) == -1 and call(dtype=3) == -1 and call(mask_dtype=9) == -1
    # config 4's sizes need a 128 MB workspace: refused with SPARTON_ESCRATCH
    assert L.sparton_fwd_workspace_bytes(32, 256, 768, 250002, 1) > cap
    assert call(B=32, S=256, D=768, V=250002) == -5
    # config 2's fit
    assert L.sparton_fwd_workspace_bytes(32, 256, 768, 30522, 1) <= cap
    assert b"static scratch" in L.sparton_strerror(-5)
