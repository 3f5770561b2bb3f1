"""The head where training/model.py puts it: a tiny BERT and a tiny XLM-R built offline from
a config (random init, no download), split into backbone, MLM transform and decoder as
_get_backbone_and_head does (training/model.py:7-45), then ProjectionSparton's calls
(training/model.py:63-85) -- SpartonMLMTransform over the transform's own parameters and
SpartonHead tied to the decoder -- against ProjectionPyTorch (training/model.py:48-60) on
the same modules, forward and backward, and the SPLADE loss on top (train.py:164-197).

Tolerances (fp32 throughout, as the reference's from_pretrained weights load):
  reps: rtol 1e-2, atol 1e-3, the head's bar.
  gradients of the projection: elementwise within 1e-3 relative plus 1e-5 of the
      gradient's largest magnitude. Both sides sum the same fp32 products in different
      orders (the transform's gelu is an erf fit within 1.2e-7 relative of torch's erf);
      torch's own fp32 CPU result sits within half this bound of float64 on these
      models, the worst case being the dense weight's gradient, whose elements are sums
      over all 192 rows with cancellation.
  near-ties: a (row, vocab) entry whose max over positions the two paths resolve to
      different positions must be a near-tie of the torch path's logits (within
      1e-4 (1 + |max|), wider than the head's own band (tests/_parity.py) since the two transforms round
      differently); such entries get a zero upstream gradient on both sides, so every
      gradient is compared in full.
  the loss and the backbone gradients through it: rtol 1e-4 on the scalars, max error
      within 1e-3 of each gradient's largest magnitude (torch's fp32 CPU result sits within
      1e-6 of float64 by this measure).
"""
import pytest
import torch
from torch import nn

import sparton_amd
from sparton_amd import loss as sl
from _parity import say

TAU = 1e-4
VOCAB, HIDDEN = 3001, 128   # ragged vocab: a partial last column tile


def tiny_mlm(kind: str, seed: int = 0):
    """A 2-layer masked LM of the reference's supported families, from its config only."""
    from transformers import BertConfig, BertForMaskedLM, XLMRobertaConfig, XLMRobertaForMaskedLM
    torch.manual_seed(seed)
    kw = dict(vocab_size=VOCAB, hidden_size=HIDDEN, num_hidden_layers=2, num_attention_heads=4,
              intermediate_size=256, attn_implementation="eager",
              hidden_dropout_prob=0.0, attention_probs_dropout_prob=0.0)  # both paths see one model
    if kind == "bert":
        return BertForMaskedLM(BertConfig(max_position_embeddings=128, **kw))
    return XLMRobertaForMaskedLM(XLMRobertaConfig(max_position_embeddings=130, **kw))


class _RobertaTransform(nn.Module):
    """dense -> gelu -> layer_norm over lm_head's own modules (training/model.py:25-34)."""

    def __init__(self, lm_head):
        super().__init__()
        self.dense, self.layer_norm = lm_head.dense, lm_head.layer_norm

    def forward(self, x):
        from transformers.activations import gelu
        return self.layer_norm(gelu(self.dense(x)))


def backbone_and_head(llm):
    """(backbone, transform, decoder) as training/model.py:7-45 extracts them."""
    if llm.config.model_type == "bert":
        p = llm.cls.predictions
        return llm.bert, p.transform, p.decoder
    return llm.roberta, _RobertaTransform(llm.lm_head), llm.lm_head.decoder


def sparton_projection(transform, decoder):
    """ProjectionSparton's construction (training/model.py:66-80): a head of the decoder's
    shape, with bias, on its device, sharing its parameters."""
    head = sparton_amd.SpartonHead(decoder.out_features, decoder.in_features, use_bias=True)
    head = head.to(device=decoder.weight.device)
    head.tie_weights(decoder)
    return sparton_amd.SpartonMLMTransform.from_hf(transform), head


def torch_projection(transform, decoder, hidden, mask):
    """ProjectionPyTorch.forward (training/model.py:56-60), also returning the positions."""
    logits = decoder(transform(hidden)) * mask.unsqueeze(-1)
    out = torch.log1p(torch.relu(logits)).max(dim=1)
    return out.values, out.indices, logits


def batch(B, S, seed, device):
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(5, VOCAB, (B, S), generator=g)
    lens = torch.randint(S // 4, S + 1, (B,), generator=g)
    lens[0] = S
    mask = (torch.arange(S)[None] < lens[:, None]).long()
    return ids.to(device), mask.to(device)


@pytest.mark.parametrize("kind", ["bert", "xlm-roberta"])
def test_projection_shares_the_models_parameters(kind):
    """CPU: the Sparton projection holds the model's own tensors (tied embeddings included),
    so an optimizer over llm.parameters() trains it."""
    llm = tiny_mlm(kind)
    _, transform, decoder = backbone_and_head(llm)
    xf, head = sparton_projection(transform, decoder)
    emb = llm.get_input_embeddings().weight
    assert head.weight is decoder.weight and head.bias is decoder.bias
    assert head.weight is emb                      # the decoder is tied to the word embeddings
    assert head.weight.shape == (VOCAB, HIDDEN)
    assert xf.dense is transform.dense
    ln = transform.LayerNorm if kind == "bert" else transform.layer_norm
    assert xf.layer_norm is ln
    own = {id(p) for p in llm.parameters()}
    assert all(id(p) in own for p in list(xf.parameters()) + list(head.parameters()))


def both_projections(transform, decoder, xf, head, h_ref, h_sp, mask):
    """Both projections on hidden states of equal value; returns (ref reps, Sparton reps,
    keep), keep being False on the entries whose gradient the two paths may route to
    different positions: a near-tie resolved differently (checked to be one), or a max so
    close to 0 that one side clamps it and the other does not."""
    ref, ref_idx, logits = torch_projection(transform, decoder, h_ref, mask)
    rep = head(xf(h_sp), mask)
    torch.testing.assert_close(rep.detach(), ref.detach(), rtol=1e-2, atol=1e-3)
    with torch.no_grad():
        _, idx = torch.ops.sparton.fused_sparton_fwd(xf(h_sp), decoder.weight, decoder.bias, mask)
        idx = idx.long()
        moved = (idx != ref_idx) & (ref > 0)
        m = logits.max(dim=1).values
        at = logits.gather(1, idx.unsqueeze(1)).squeeze(1)
        assert bool((at[moved] >= m[moved] - TAU * (1 + m[moved].abs())).all()), "not a near-tie"
        keep = ~moved & ((ref > 0) == (rep > 0))
    say(f"  positive entries {int((ref > 0).sum())}, entries left out {int((~keep).sum())}")
    return ref, rep, keep


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["bert", "xlm-roberta"])
def test_projection_matches_torch_projection(kind, device):
    say(f"hf projection {kind}")
    llm = tiny_mlm(kind, seed=1).to(device)
    backbone, transform, decoder = backbone_and_head(llm)
    ids, mask = batch(4, 48, seed=2, device=device)
    with torch.no_grad():
        hidden = backbone(ids, mask).last_hidden_state
    xf, head = sparton_projection(transform, decoder)
    h_ref, h_sp = hidden.clone().requires_grad_(), hidden.clone().requires_grad_()
    ref, rep, keep = both_projections(transform, decoder, xf, head, h_ref, h_sp, mask)

    G = torch.rand(ref.shape, generator=torch.Generator().manual_seed(3)).to(device) * keep
    params = [transform.dense.weight, transform.dense.bias, xf.layer_norm.weight,
              xf.layer_norm.bias, decoder.weight, decoder.bias]
    g_ref = torch.autograd.grad(ref, [h_ref] + params, G)
    g_sp = torch.autograd.grad(rep, [h_sp] + params, G)
    names = ["hidden", "dense W", "dense b", "LN weight", "LN bias", "decoder W", "decoder b"]
    for a, r, n in zip(g_sp, g_ref, names):
        assert a.dtype == torch.float32 and a.shape == r.shape, n
        atol = 1e-5 * r.abs().max().item()
        torch.testing.assert_close(a, r, rtol=1e-3, atol=atol, msg=lambda s: f"{n}: {s}")


@pytest.mark.gpu
def test_projection_under_bf16_autocast(device):
    """Mixed precision as a Trainer's bf16 autocast runs it: bf16 reps from the fp32 model,
    within bf16 rounding of the fp32 torch projection (max error vs max magnitude)."""
    llm = tiny_mlm("bert", seed=4).to(device)
    backbone, transform, decoder = backbone_and_head(llm)
    ids, mask = batch(4, 32, seed=5, device=device)
    with torch.no_grad():
        hidden = backbone(ids, mask).last_hidden_state
        ref = torch_projection(transform, decoder, hidden, mask)[0]
    xf, head = sparton_projection(transform, decoder)
    h = hidden.clone().requires_grad_()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        rep = head(xf(h), mask)
    assert rep.dtype == torch.bfloat16
    err = (rep.float() - ref).abs().max().item()
    assert err <= 3e-2 * ref.abs().max().item(), err
    rep.float().sum().backward()
    assert decoder.weight.grad.dtype == torch.float32 and torch.isfinite(decoder.weight.grad).all()
    assert h.grad is not None and torch.isfinite(h.grad).all()


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["bert", "xlm-roberta"])
def test_training_step_matches_torch_head(kind, device):
    """SpladeModel's sparton path end to end (training/model.py:124-139, train.py:164-197):
    backbone -> projection -> SPLADE loss -> backward into every model parameter, against
    the same model with the torch projection and the reference's loss formulas."""
    say(f"hf training step {kind}")
    llm = tiny_mlm(kind, seed=6).to(device)
    backbone, transform, decoder = backbone_and_head(llm)
    xf, head = sparton_projection(transform, decoder)
    q_ids, q_mask = batch(8, 16, seed=7, device=device)
    d_ids, d_mask = batch(8, 64, seed=8, device=device)
    T, w_l1, w_fl = 100.0, 1e-3, 1e-3   # scores of a random model are ~600: T keeps the softmax soft
    params = [p for p in llm.parameters() if p.requires_grad]

    def encode(ids, mask):
        """Both paths from one backbone pass each; the entries both leave out get no
        gradient on either side (a hook on each reps tensor)."""
        h_ref = backbone(ids, mask).last_hidden_state
        h_sp = backbone(ids, mask).last_hidden_state
        ref, rep, keep = both_projections(transform, decoder, xf, head, h_ref, h_sp, mask)
        for r in (ref, rep):
            r.register_hook(lambda g: g * keep)
        return ref, rep

    def ref_loss(q, d):
        s = q @ d.t() / T
        ce = nn.functional.cross_entropy(s, torch.arange(q.shape[0], device=device))
        l1 = q.abs().sum(-1).mean() + d.abs().sum(-1).mean()
        fl = (q.sum(0) ** 2).mean() + (d.sum(0) ** 2).mean()
        return ce + w_l1 * l1 + w_fl * fl

    (q_ref, q_sp), (d_ref, d_sp) = encode(q_ids, q_mask), encode(d_ids, d_mask)
    llm.zero_grad()
    lr = ref_loss(q_ref, d_ref)
    lr.backward()
    g_ref = [None if p.grad is None else p.grad.clone() for p in params]
    llm.zero_grad()
    res = sl.splade_loss(q_sp, d_sp, T, w_l1, w_fl)
    res.total.backward()
    torch.testing.assert_close(res.total, lr.detach(), rtol=1e-4, atol=1e-6)
    # The attention key biases get gradients that are 0 up to roundoff (softmax ignores a
    # shift shared by a row), so each scale has a floor of 1e-4 of the largest gradient.
    floor = 1e-4 * max(r.abs().max().item() for r in g_ref if r is not None)
    worst = 0.0
    for p, r in zip(params, g_ref):
        assert (p.grad is None) == (r is None)
        if r is not None:
            worst = max(worst, (p.grad - r).abs().max().item() / max(r.abs().max().item(), floor))
    say(f"  loss {res.total.item():.6f} (torch {lr.item():.6f}), worst grad rel err {worst:.2e}")
    assert worst <= 1e-3


@pytest.mark.gpu
def test_projection_compiles_fullgraph(device):
    """torch.compile(fullgraph=True) over the Sparton projection (the transform's and the
    head's custom ops, with their fakes and autograd): the same kernels as eager, so the
    reps and every gradient are bitwise equal."""
    llm = tiny_mlm("bert", seed=9).to(device)
    backbone, transform, decoder = backbone_and_head(llm)
    xf, head = sparton_projection(transform, decoder)
    ids, mask = batch(2, 24, seed=10, device=device)
    with torch.no_grad():
        hidden = backbone(ids, mask).last_hidden_state

    def proj(h, m):
        return head(xf(h), m)

    compiled = torch.compile(proj, backend="aot_eager", fullgraph=True)
    G = torch.rand(2, VOCAB, generator=torch.Generator().manual_seed(11)).to(device)
    params = [transform.dense.weight, transform.dense.bias, decoder.weight, decoder.bias]
    outs = []
    for fn in (proj, compiled):
        h = hidden.clone().requires_grad_()
        r = fn(h, mask)
        outs.append([r.detach()] + list(torch.autograd.grad(r, [h] + params, G)))
    for a, b in zip(*outs):
        assert torch.equal(a, b)
