"""CPU oracle vs what the mathematics fixes.

For the oracle functions the reference CPU runtime does not have (RMSNorm
and its backward with the optional gain, the attention chain and its
backward, cross-entropy, the whole GPT training step) these checks pin the
oracle independently of its own formulas:
  * closed forms evaluated in float64 (CE = logsumexp - x_t, attention as
    softmax(QK^T/8 + mask)V written directly in numpy);
  * invariants (softmax rows sum to 1, CE gradient rows sum to 0);
  * central finite differences of the forward for every backward, so a
    dropped term, a wrong sign or a transposed operand fails.
"""
import numpy as np
import pytest

import oracle_lib as O


def rel_err(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / (np.max(np.abs(b)) + 1e-30))


def test_softmax_rows_sum_to_one():
    x = O.normal((50, 333), 11, 0, 5)
    y = O.softmax(x)
    np.testing.assert_allclose(y.sum(axis=1), 1.0, rtol=0, atol=2e-6)
    assert np.all(y >= 0)


def test_cross_entropy_closed_form_and_grad_invariant():
    logits = O.normal((40, 97), 12, 0, 3)
    t = O.uniform_u32((40,), 13, 97)
    x = logits.astype(np.float64)
    m = x.max(axis=1, keepdims=True)
    lse = (m + np.log(np.exp(x - m).sum(axis=1, keepdims=True)))[:, 0]
    expect = lse - x[np.arange(40), t]
    assert rel_err(O.cross_entropy(logits, t)[:, 0], expect) < 1e-6
    g = O.cross_entropy_backward(logits, t)
    np.testing.assert_allclose(g.sum(axis=1), 0.0, atol=1e-6)
    p = np.exp(x - lse[:, None])
    p[np.arange(40), t] -= 1
    assert rel_err(g, p) < 1e-5


def _rmsnorm64(x, gain, eps):
    x = x.astype(np.float64)
    r = np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
    y = x / r
    return y * gain if gain is not None else y


@pytest.mark.parametrize("with_gain", [False, True])
def test_rms_norm_forward_closed_form(with_gain):
    x = O.normal((20, 48), 14)
    gain = O.normal((48,), 15, 1, 0.02) if with_gain else None
    y = O.rms_norm(x, gain, eps=1e-5)
    assert rel_err(y, _rmsnorm64(x, gain, 1e-5)) < 1e-6


@pytest.mark.parametrize("with_gain", [False, True])
def test_rms_norm_backward_finite_differences(with_gain):
    rows, cols, eps = 4, 12, 1e-6
    x = O.normal((rows, cols), 16).astype(np.float64)
    gain = O.normal((cols,), 17, 1, 0.2).astype(np.float64) if with_gain else None
    g = O.normal((rows, cols), 18).astype(np.float64)
    dx, dgain = O.rms_norm_backward(g.astype(np.float32), x.astype(np.float32),
                                    None if gain is None else gain.astype(np.float32), eps)
    h = 1e-6
    num = np.zeros_like(x)
    for i in range(rows):
        for j in range(cols):
            xp = x.copy(); xp[i, j] += h
            xm = x.copy(); xm[i, j] -= h
            num[i, j] = ((_rmsnorm64(xp, gain, eps) - _rmsnorm64(xm, gain, eps)) * g).sum() / (2 * h)
    assert rel_err(dx, num) < 1e-4
    if with_gain:
        n = _rmsnorm64(x, None, eps)
        assert rel_err(dgain, (g * n).sum(axis=0)) < 1e-5


def _attention64(q, k, v, causal):
    q, k, v = (a.astype(np.float64) for a in (q, k, v))
    s = q @ np.swapaxes(k, -1, -2) / np.sqrt(q.shape[-1])
    if causal:
        T = q.shape[-2]
        s = s + np.triu(np.full((T, T), -np.inf), 1)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return p @ v, p


@pytest.mark.parametrize("causal", [True, False])
def test_attention_forward_closed_form(causal):
    B, H, T, D = 2, 3, 17, 8
    q, k, v = (O.normal((B, H, T, D), s, 0, 1) for s in (20, 21, 22))
    o, probs = O.attention_forward(q, k, v, causal)
    o64, p64 = _attention64(q, k, v, causal)
    assert rel_err(o, o64) < 1e-5
    assert rel_err(probs, p64) < 1e-5


def test_attention_backward_finite_differences():
    B, H, T, D = 1, 2, 6, 4
    q, k, v = (O.normal((B, H, T, D), s, 0, 1).astype(np.float64) for s in (23, 24, 25))
    dout = O.normal((B, H, T, D), 26).astype(np.float64)
    _, probs = O.attention_forward(q, k, v, True)
    dq, dk, dv = O.attention_backward(q, k, v, probs, dout)

    def loss(qq, kk, vv):
        return (_attention64(qq, kk, vv, True)[0] * dout).sum()

    h = 1e-6
    for arr, grad in ((q, dq), (k, dk), (v, dv)):
        num = np.zeros_like(arr)
        it = np.nditer(arr, flags=["multi_index"])
        for _ in it:
            idx = it.multi_index
            old = arr[idx]
            arr[idx] = old + h
            lp = loss(q, k, v)
            arr[idx] = old - h
            lm = loss(q, k, v)
            arr[idx] = old
            num[idx] = (lp - lm) / (2 * h)
        assert rel_err(grad, num) < 1e-4


# ---- GPT training step -------------------------------------------------------
TINY = dict(vocab=11, seq=5, dim=8, heads=2, layers=2, batch=2, ffn=12)


def _tiny_setup(seed=30):
    cfg = O.gpt_config(**TINY)
    sizes = O.gpt_param_sizes(cfg)
    total = sum(sizes)
    params = O.normal((total,), seed, 0, 0.3)
    tokens = O.uniform_u32((TINY["batch"] * TINY["seq"],), seed + 1, TINY["vocab"])
    targets = O.uniform_u32((TINY["batch"] * TINY["seq"],), seed + 2, TINY["vocab"])
    return cfg, sizes, params, tokens, targets


def _loss(cfg, params, tokens, targets, root):
    logits = O.gpt_forward(cfg, params.astype(np.float32), tokens).astype(np.float64)
    m = logits.max(axis=1, keepdims=True)
    lse = (m + np.log(np.exp(logits - m).sum(axis=1, keepdims=True)))[:, 0]
    return float(root * (lse - logits[np.arange(len(targets)), targets]).sum())


def test_gpt_gradients_finite_differences():
    """Directional derivative of the loss along a random direction per
    parameter tensor vs <grad, direction> from the hand-written backward."""
    cfg, sizes, params, tokens, targets = _tiny_setup()
    root = 1.0 / len(tokens)
    z = np.zeros_like(params)
    out = O.gpt_train_step(cfg, params, z, z, 1, tokens, targets, root, 0, 0.9, 0.95, 1e-8, 0,
                           0.0)
    grads = out["grads"].astype(np.float64)
    base_loss = root * float(out["losses"].astype(np.float64).sum())
    assert abs(base_loss - _loss(cfg, params, tokens, targets, root)) < 1e-5
    rng = np.random.default_rng(0)
    off = 0
    h = 1e-2
    for i, n in enumerate(sizes):
        d = np.zeros_like(params, dtype=np.float64)
        d[off:off + n] = rng.standard_normal(n)
        analytic = float((grads * d).sum())
        lp = _loss(cfg, params + h * d, tokens, targets, root)
        lm = _loss(cfg, params - h * d, tokens, targets, root)
        numeric = (lp - lm) / (2 * h)
        scale = max(abs(analytic), abs(numeric), 1e-4)
        assert abs(analytic - numeric) / scale < 2e-2, (i, analytic, numeric)
        off += n


def test_gpt_step_clip_and_adamw_closed_form():
    """One step = global-norm clip + AdamW (compile.h:236-258, AdamW.h)."""
    cfg, sizes, params, tokens, targets = _tiny_setup(40)
    root = 1.0 / len(tokens)
    z = np.zeros_like(params)
    lr, b1, b2, eps, wd, max_norm = 1e-2, 0.9, 0.95, 1e-8, 0.1, 0.05
    out = O.gpt_train_step(cfg, params, z, z, 1, tokens, targets, root, lr, b1, b2, eps, wd,
                           max_norm)
    g = out["grads"].astype(np.float64)
    sq = float((g * g).sum())
    assert abs(out["squared_norm"] - sq) / sq < 1e-5
    scale = min(1.0, max_norm / np.sqrt(sq))
    gc = g * scale
    m = (1 - b1) * gc
    v = (1 - b2) * gc * gc
    decay = np.float32(1) - np.float32(lr) * np.float32(wd)
    expect = params * np.float64(decay) - lr * (m / (1 - b1)) / (np.sqrt(v / (1 - b2)) + eps)
    assert rel_err(out["params"], expect) < 1e-5
    assert rel_err(out["m"], m) < 1e-5 and rel_err(out["v"], v) < 1e-5
