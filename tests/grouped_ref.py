"""Expected output of the batched (grouped) path for one token.

The batched router computes every logit as the reference does (the serial
fp32 chain acc = b; acc += W[j] * xn[j], engine_gpt2.rs:849-852,
engine_qwen2.rs:395-400), so the batched selection is the reference's: its
experts, their rank order and their softmax weights are the oracle's router
+ top-k on the token's xn.  The experts' down rows (+ bias) are per-token
decode's, whose integer block sums the tests compare bit for bit.  The
combine is x += w_s * (down_s + b) over the reference's slots in order, in
fp32 (engine_gpt2.rs:911-921, engine_qwen2.rs:426-432).

The weights go through expf on the GPU and in the oracle; the two may differ
by an ulp, which moves an output by ~1e-7 of its RMS.  So a batch is checked
as: every token within 4e-6 of the output RMS, and most tokens (at least
60 %) bit for bit.  Per-token decode's weights (softmax of its fp64 interval
centres rounded to fp32) miss the reference's on every token by 4e-7 to
1e-6 of the RMS and match none bit for bit, so the second condition is what
pins the batched weights to the reference's logits.
"""
import numpy as np

from oracle import oracle as O


def grouped_expect(L, x, tr, family):
    """L: the layer dict; x: the token's input; tr: per-token decode's trace
    of the same token.  Returns (expected output, reference ids, decode slot
    of each reference slot)."""
    d, ne, k = L["d"], L["ne"], L["k"]
    W = np.asarray(L["router_w"], np.float32).reshape(ne, d)
    logits = O.router(W, L.get("router_b"), tr["xn"])
    ids, w = (O.topk_gptoss if family == "gptoss" else O.topk_qwen)(logits, k)
    slot = {int(e): s for s, e in enumerate(tr["ids"])}
    assert sorted(slot) == sorted(int(e) for e in ids), ("decode and reference selections differ", tr["ids"], ids)
    order = [slot[int(e)] for e in ids]
    acc = np.array(x, np.float32)
    for s in range(k):
        acc = acc + np.float32(w[s]) * tr["dn"][order[s]]
    return acc.astype(np.float32), ids, order


class BatchCheck:
    """Accumulates grouped_expect comparisons of one batch."""

    def __init__(self):
        self.n = 0
        self.exact = 0

    def add(self, y, ye, x, where):
        rms = np.sqrt(((ye - x).astype(np.float64) ** 2).mean())
        err = float(np.max(np.abs(y.astype(np.float64) - ye)))
        assert err <= 4e-6 * rms, ("grouped output off the reference combine", where, err / rms)
        self.n += 1
        self.exact += int(np.array_equal(y.view(np.uint32), ye.view(np.uint32)))

    def done(self):
        # the bit-exact share says something only over enough tokens
        if self.n >= 10:
            assert self.exact >= 0.6 * self.n, ("too few tokens bit-exact to the reference combine", self.exact, self.n)
