"""The oracle's restatement of DecisionModel.ReadOut (src/StructuredDecisions.Laya/Models/DecisionModel.cs:170-226),
pinned without the reference's runtime: an independent float64 formulation in numpy of the same read-out
from the same pooled rows and logits, and closed forms (uniform logits: p = 1/K, normalised entropy 1 for
K ≥ 2 and 0 for K = 1, margin 0; the K/255 feature)."""
import numpy as np
from scipy.special import erf

import oracle
from fixtures import TINY, tiny_batch, tiny_config, tiny_params


def _numpy_readout(logits, n_options, pooled, P):
    """The read-out in float64 numpy, written from DecisionModel.ReadOut's text."""
    probs, feats = [], []
    off = 0
    for i, K in enumerate(n_options):
        z = np.asarray(logits[off:off + K], np.float64)
        off += K
        p = np.exp(z - z.max())
        p /= p.sum()
        k = max(2, K)
        ent = -np.sum(p * np.log(np.maximum(p, 1e-9))) / np.log(k)
        srt = np.sort(p)[::-1]
        top1, top2 = srt[0], (srt[1] if K > 1 else 0.0)
        x = np.concatenate([pooled[i], [top1, top1 - top2, ent, k / 255.0]])
        h = P["act_head.0.weight"].astype(np.float64) @ x + P["act_head.0.bias"]
        h = 0.5 * h * (1.0 + erf(h / np.sqrt(2.0)))
        a = P["act_head.2.weight"].astype(np.float64) @ h + P["act_head.2.bias"]
        a = np.exp(a - a.max())
        probs.append(a / a.sum())
        feats.append([top1, top1 - top2, ent, k / 255.0])
    return np.array(probs), np.array(feats)


def test_readout_matches_an_independent_formulation():
    params = tiny_params()  # the fixture's act head weights
    batch, _, _ = tiny_batch()
    for double in (True, False):
        o = oracle.OracleModel(tiny_config(), double=double)
        o.set_params(params)
        logits = o.forward(batch, training=False)
        probs, feats, pooled = o.readout()
        want_p, want_f = _numpy_readout(logits, batch.n_options, pooled, params)
        tol = 2e-7 if double else 2e-6  # the outputs are float32
        np.testing.assert_allclose(feats, want_f, rtol=tol, atol=tol)
        np.testing.assert_allclose(probs, want_p, rtol=tol * 10, atol=tol)
        np.testing.assert_allclose(probs.sum(axis=1), 1.0, atol=1e-6)


def test_uniform_logits_give_the_closed_form_features():
    params = tiny_params()
    params["scorer.3.weight"] = np.zeros_like(params["scorer.3.weight"])  # every logit = the output bias
    o = oracle.OracleModel(tiny_config(), double=True)
    o.set_params(params)
    batch, _, _ = tiny_batch()
    o.forward(batch, training=False)
    _, feats, _ = o.readout()
    for i, K in enumerate(batch.n_options):
        assert abs(feats[i, 0] - 1.0 / K) < 1e-7
        assert abs(feats[i, 1]) < 1e-7
        assert abs(feats[i, 2] - (1.0 if K >= 2 else 0.0)) < 1e-6
        assert abs(feats[i, 3] - max(2, K) / 255.0) < 1e-7


def test_act_head_reads_the_pooled_row_and_features_in_order():
    """Closed form: with the act head wired to pass one input slot through GELU to action logit 0 (logit 1 is
    GELU(0) = 0), log(p0/p1) = GELU(slot value) for pooled columns 0, 1, 17, 63 of h[start] and the four
    features, whose values are known without the read-out's formulas (tests/helpers.closed_form_readout_case).
    A pooled row other than the item's first (its column 0 has the other sign), a pooled value taken before the
    type embedding, or features in another order all fail."""
    from helpers import READOUT_SLOTS, act_head_selecting, closed_form_readout_case
    mc, params, batch, expected = closed_form_readout_case()
    for double in (True, False):
        for slot in READOUT_SLOTS:
            o = oracle.OracleModel(mc, double=double)
            o.set_params(act_head_selecting(params, slot))
            o.forward(batch, training=False)
            probs, feats, _ = o.readout()
            got = np.log(probs[:, 0].astype(np.float64) / probs[:, 1])
            x = expected[:, slot]
            want = 0.5 * x * (1.0 + erf(x / np.sqrt(2.0)))
            np.testing.assert_allclose(got, want, atol=2e-6, err_msg=f"slot {slot}")
        np.testing.assert_allclose(feats, expected[:, 64:], atol=1e-6)
