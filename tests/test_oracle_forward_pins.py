"""Closed-form pins of the oracle's forward composition (src/forward.rs:375-505):
which norm weight, bias, residual and operand goes where (CPU only).

The reference checks its forward only against candle
(examples/compare_forward.rs), which is not available here. These models are
special cases whose logits follow from the architecture's definition in a
few lines of float64, independent of the oracle's code:

- o-proj and down all zero: every layer is the identity on the residual, so
  logits = W_out . rmsnorm(embd[last], output_norm);
- o-proj zero: only the SwiGLU block of each layer changes the residual;
- v weights zero: every cached V row is the v bias, so each head's
  attention output is its KV group's bias whatever the scores are;
- q and k weights zero: the scores come from the rotated biases alone, and
  the positions of the rotation can be read off them.

The matrices are F32, the path matmul_auto takes for unquantized weights
(ops::matmul, src/ops.rs:87-156), so no activation quantization enters and
the f32 forward agrees with float64 to ~1e-6. Norm weights, biases and
embeddings differ per tensor, so swapping any two of them changes the
result. tests/test_oracle_mutants.py compiles plausible slips into copies of
the oracle and shows that these tests fail on each."""
import math

import numpy as np
import pytest

from oracle import oracle as O

CFG = dict(layers=1, dim=64, heads=4, kv_heads=2, ffn=96, vocab=40, ctx=32, eps=1e-6,
           rope_base=10000.0)


def _rms(x, w, eps):
    """src/kernels/scalar.rs:36-54: x / sqrt(mean(x^2) + eps) * w."""
    x = np.asarray(x, np.float64)
    return x / math.sqrt(float(np.mean(x * x)) + eps) * np.asarray(w, np.float64)


def _silu(z):
    """src/kernels/scalar.rs:63-67."""
    return z / (1.0 + np.exp(-z))


def _rope(v, pos, base):
    """src/ops.rs:1150-1193: value i turns against i + d/2 by pos * base^(-2i/d)."""
    hd = v.size
    half = hd // 2
    th = pos * base ** (-2.0 * np.arange(half) / hd)
    a, b = v[:half], v[half:]
    return np.concatenate([a * np.cos(th) - b * np.sin(th), a * np.sin(th) + b * np.cos(th)])


def _model(cfg, seed, zero=(), identity=(), sigma=0.2):
    """Host tensors of a qwen2 model with F32 matrices: embeddings N(0, 1),
    norms N(1, 0.2) and biases N(0, 0.5), a draw per tensor; matrices
    N(0, sigma) except those named in `zero` (all 0) and `identity`."""
    rng = np.random.default_rng(seed)
    D, I, V = cfg["dim"], cfg["ffn"], cfg["vocab"]
    kvd = cfg["kv_heads"] * D // cfg["heads"]
    t, ty = {}, {}

    def mat(name, rows, cols):
        short = name.split(".")[-2]
        if short in zero:
            a = np.zeros((rows, cols))
        elif short in identity:
            a = np.eye(rows, cols)
        else:
            a = rng.normal(0, sigma, (rows, cols))
        t[name], ty[name] = a.astype(np.float32), O.F32

    def vec(name, n, mean, sd):
        t[name], ty[name] = rng.normal(mean, sd, n).astype(np.float32), O.F32

    vec("token_embd.weight", V * D, 0.0, 1.0)
    for i in range(cfg["layers"]):
        p = f"blk.{i}."
        vec(p + "attn_norm.weight", D, 1.0, 0.2)
        vec(p + "ffn_norm.weight", D, 1.0, 0.2)
        for b, n in (("attn_q.bias", D), ("attn_k.bias", kvd), ("attn_v.bias", kvd)):
            vec(p + b, n, 0.0, 0.5)
        mat(p + "attn_q.weight", D, D)
        mat(p + "attn_k.weight", kvd, D)
        mat(p + "attn_v.weight", kvd, D)
        mat(p + "attn_output.weight", D, D)
        mat(p + "ffn_gate.weight", I, D)
        mat(p + "ffn_up.weight", I, D)
        mat(p + "ffn_down.weight", D, I)
    vec("output_norm.weight", D, 1.0, 0.2)
    mat("output.weight", V, D)
    return t, ty


def _f64(t, name):
    return t[name].astype(np.float64)


def _logits(t, cfg, x):
    return _f64(t, "output.weight") @ _rms(x, _f64(t, "output_norm.weight"), cfg["eps"])


def _run(t, ty, cfg, prompt, steps):
    """The oracle's logits after the prompt and after each single-token step."""
    m = O.Model(cfg, t, ty, threads=2)
    c = m.new_cache(cfg["ctx"])
    out = [m.forward(np.array(prompt, np.uint32), c)]
    for tok in steps:
        out.append(m.forward(np.array([tok], np.uint32), c))
    return out


def _close(got, want, what):
    want = np.asarray(want, np.float64)
    err = float(np.max(np.abs(got - want)))
    assert err <= 1e-5 * float(np.max(np.abs(want))) + 1e-7, (what, err, float(np.max(np.abs(want))))


def _embd(t, cfg, tok):
    D = cfg["dim"]
    return _f64(t, "token_embd.weight")[tok * D:(tok + 1) * D]


@pytest.mark.parametrize("layers", [1, 2])
def test_identity_layers_leave_the_output_norm_and_head(layers):
    """o-proj and down zero: x stays the token's embedding through every
    layer (src/forward.rs:467-469, 489-491 add zero), so the logits are
    W_out . rmsnorm(embd[last token], output_norm) (495-501), whatever the
    attention, the norms of the layers and the SwiGLU compute."""
    cfg = dict(CFG, layers=layers)
    t, ty = _model(cfg, 10 + layers, zero=("attn_output", "ffn_down"))
    prompt, steps = [3, 7, 11, 5], [9, 2]
    got = _run(t, ty, cfg, prompt, steps)
    for g, last in zip(got, [prompt[-1]] + steps):
        _close(g, _logits(t, cfg, _embd(t, cfg, last)), ("token", last))


def test_swiglu_block_closed_form():
    """o-proj zero: the layer is x + W_down . (silu(W_gate . n) * (W_up . n))
    with n = rmsnorm(x, ffn_norm) (src/forward.rs:472-491), then the final
    norm and head; attn_norm, ffn_norm and output_norm are distinct."""
    cfg = CFG
    t, ty = _model(cfg, 21, zero=("attn_output",))
    prompt, steps = [4, 8, 15], [16, 23]
    got = _run(t, ty, cfg, prompt, steps)
    for g, last in zip(got, [prompt[-1]] + steps):
        x = _embd(t, cfg, last)
        n = _rms(x, _f64(t, "blk.0.ffn_norm.weight"), cfg["eps"])
        h = _silu(_f64(t, "blk.0.ffn_gate.weight") @ n) * (_f64(t, "blk.0.ffn_up.weight") @ n)
        _close(g, _logits(t, cfg, x + _f64(t, "blk.0.ffn_down.weight") @ h), ("token", last))


def test_attention_of_constant_values_is_the_group_bias():
    """v weights zero and down zero: every cached V row is the v bias
    (src/forward.rs:428-436), the softmax weights sum to 1, so head h's
    attention output is the bias of its KV group h / (heads / kv_heads)
    (src/ops.rs:1258-1325), and x = embd + W_o . [bias of each head's group]
    (src/forward.rs:465-469). The groups' biases differ."""
    cfg = CFG
    t, ty = _model(cfg, 33, zero=("attn_v", "ffn_down"))
    hd = cfg["dim"] // cfg["heads"]
    per = cfg["heads"] // cfg["kv_heads"]
    bv = _f64(t, "blk.0.attn_v.bias")
    att = np.concatenate([bv[(h // per) * hd:(h // per + 1) * hd] for h in range(cfg["heads"])])
    prompt, steps = [1, 2, 3, 4, 5], [6, 7]
    got = _run(t, ty, cfg, prompt, steps)
    for g, last in zip(got, [prompt[-1]] + steps):
        x = _embd(t, cfg, last) + _f64(t, "blk.0.attn_output.weight") @ att
        _close(g, _logits(t, cfg, x), ("token", last))


def test_scores_from_rotated_biases():
    """q and k weights zero: the query at position p is the q bias rotated
    by p, the key at position j the k bias rotated by j (src/forward.rs:
    428-452, the rotation at the cache's length plus the token's index);
    scores are their dot over sqrt(head_dim), a causal softmax weighs the
    values W_v . rmsnorm(embd, attn_norm) + v bias of positions 0..p
    (src/ops.rs:1258-1325). With o-proj the identity and down zero,
    x = embd[last] + attention output."""
    cfg = CFG
    t, ty = _model(cfg, 44, zero=("attn_q", "attn_k", "ffn_down"), identity=("attn_output",))
    t["blk.0.attn_q.bias"] = np.random.default_rng(5).normal(0, 1.5, cfg["dim"]).astype(np.float32)
    D, hd = cfg["dim"], cfg["dim"] // cfg["heads"]
    per = cfg["heads"] // cfg["kv_heads"]
    kvd = cfg["kv_heads"] * hd
    t["blk.0.attn_k.bias"] = np.random.default_rng(6).normal(0, 1.5, kvd).astype(np.float32)
    bq, bk = _f64(t, "blk.0.attn_q.bias"), _f64(t, "blk.0.attn_k.bias")
    wv, bv = _f64(t, "blk.0.attn_v.weight"), _f64(t, "blk.0.attn_v.bias")
    an = _f64(t, "blk.0.attn_norm.weight")
    prompt, steps = [9, 3, 30, 12, 7, 21], [5, 38]
    toks = prompt + steps
    vals = [wv @ _rms(_embd(t, cfg, tk), an, cfg["eps"]) + bv for tk in toks]
    got = _run(t, ty, cfg, prompt, steps)
    for g, p in zip(got, [len(prompt) - 1] + [len(prompt) + i for i in range(len(steps))]):
        att = np.zeros(D)
        for h in range(cfg["heads"]):
            gr = h // per
            q = _rope(bq[h * hd:(h + 1) * hd], p, cfg["rope_base"])
            sc = np.array([q @ _rope(bk[gr * hd:(gr + 1) * hd], j, cfg["rope_base"])
                           for j in range(p + 1)]) / math.sqrt(hd)
            w = np.exp(sc - sc.max())
            w /= w.sum()
            att[h * hd:(h + 1) * hd] = sum(w[j] * vals[j][gr * hd:(gr + 1) * hd]
                                           for j in range(p + 1))
        _close(g, _logits(t, cfg, _embd(t, cfg, toks[p]) + att), ("position", p))
