"""The error bound of the fp32 split mode (torch's 'high' float32 matmul precision), which the
GPU parity band uses: with hi = bf16(x) and lo = bf16(x - hi) (round to nearest even, as
v_cvt_pk_bf16_f32 and torch's bfloat16 cast do), x - hi is exact in fp32,
|x - hi - lo| <= 2^-16 |x|, and a product taken as hi_a hi_b + hi_a lo_b + lo_a hi_b is within
3 * 2^-16 |a b| of the exact one. Checked in float64 on random values over a wide exponent
range, with a planted mistake (the hi_a lo_b term dropped) that the bound must reject."""
import torch

from _parity import SPLIT_REL


def split(x):
    hi = x.to(torch.bfloat16).to(torch.float32)
    r = x - hi  # exact in fp32
    lo = r.to(torch.bfloat16).to(torch.float32)
    return hi, lo, r


def sample(n, seed):
    g = torch.Generator().manual_seed(seed)
    mant = torch.rand(n, generator=g, dtype=torch.float64) + 1.0
    expo = torch.randint(-60, 60, (n,), generator=g).to(torch.float64)
    sign = torch.where(torch.rand(n, generator=g) < 0.5, -1.0, 1.0).to(torch.float64)
    return (sign * mant * torch.pow(2.0, expo)).to(torch.float32)


def test_remainder_is_exact_and_within_2_pow_minus_16():
    x = sample(200000, 1)
    hi, lo, r = split(x)
    xd, hid, lod = x.double(), hi.double(), lo.double()
    assert torch.equal(r.double(), xd - hid)  # x - hi needs no rounding
    assert bool(((xd - hid - lod).abs() <= 2.0 ** -16 * xd.abs()).all())
    assert bool(((xd - hid).abs() <= 2.0 ** -8 * xd.abs()).all())


def test_split_product_within_split_rel():
    a, b = sample(200000, 2), sample(200000, 3)
    ha, la, _ = split(a)
    hb, lb, _ = split(b)
    exact = a.double() * b.double()
    got = ha.double() * hb.double() + ha.double() * lb.double() + la.double() * hb.double()
    assert SPLIT_REL == 3 * 2.0 ** -16
    err = (got - exact).abs()
    assert bool((err <= SPLIT_REL * exact.abs()).all()), float((err / exact.abs()).max())
    # the bound is not loose by orders of magnitude: the worst case reaches a good part of it
    assert float((err / exact.abs()).max()) > 2.0 ** -17
    # a dropped cross term breaks it
    bad = ha.double() * hb.double() + la.double() * hb.double()
    assert not bool(((bad - exact).abs() <= SPLIT_REL * exact.abs()).all())
