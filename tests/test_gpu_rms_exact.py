"""RMSNorm is bit-exact, not probably exact (GPU, through the C ABI).

The reference sums the squares in f64 in order (src/kernels/scalar.rs:47);
the GPU sums them as a workgroup tree, bounds how far that can be from the
sum in order, and sums again in order whenever some output's f32 could
round differently within the bound. The vectors here (tests/rms_fixtures.py)
are built so that both of the GPU's trees do round one output differently
from the sum in order, and that output is the amax of its 32-value
sub-block, so that the quantized activation and everything after it would
change. Every site that normalizes sees one: cx_rmsnorm; the decode step's
q/k/v, gate/up and final norms; the prefill's; at widths 2048 (the row
kernels), 4096 (config 5's) and 896 (the Q8_0 kernels). Bars: outputs and
logits bit-identical to the oracle's."""
import numpy as np
import pytest
import torch

import rms_fixtures as R
from gguf_fixtures import mirror, write_tensor
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [2048, 4096, 896, 1024])
def test_rmsnorm_operator_on_splitting_vectors(dev, n):
    from cosxamix_amd import ops
    rows = []
    for seed in range(3):
        x, j = R.splitting_vector(n, seed)
        s = R.seq_sum(x)
        # the teeth: the operator's tree alone would give another f32 at j
        assert R.f32_of(x[j], R.factor(R.tree4_sum(x), n, 1e-6)) != R.f32_of(x[j], R.factor(s, n, 1e-6))
        rows.append(x)
    x = np.stack(rows)
    w = np.random.default_rng(n).normal(1.0, 0.1, n).astype(np.float32)
    out = torch.empty(3 * n, device=dev)
    ops.rmsnorm(out, torch.from_numpy(x.ravel()).to(dev), torch.from_numpy(w).to(dev), 1e-6)
    got = out.cpu().numpy().reshape(3, n)
    for r in range(3):
        want = O.rmsnorm(x[r], w, 1e-6)
        assert np.array_equal(got[r].view(np.uint32), want.view(np.uint32)), r


CASES = [
    ("2048-q4k", dict(capas=1, dim=2048, cabezas=16, cabezas_kv=2, ffn=1024, vocab=300,
                      contexto=64), O.Q4_K, O.Q4_K),
    ("4096-q4k-q5kdown", dict(capas=1, dim=4096, cabezas=32, cabezas_kv=8, ffn=2048, vocab=300,
                              contexto=64, rope=5e5), O.Q4_K, O.Q5_K),
    ("896-q8_0", dict(capas=1, dim=896, cabezas=14, cabezas_kv=2, ffn=1024, vocab=300,
                      contexto=64), O.Q8_0, O.Q8_0),
]
# which norm sees the constructed residual: o-proj zero passes it on to the
# ffn norm, o-proj and down zero to the final norm
STAGES = {"attn_norm": (), "ffn_norm": ("attn_output",), "output_norm": ("attn_output", "ffn_down")}


@pytest.mark.parametrize("stage", list(STAGES))
@pytest.mark.parametrize("name,cfg,t,tdown", CASES, ids=[c[0] for c in CASES])
def test_model_norms_on_splitting_vectors(dev, name, cfg, t, tdown, stage):
    from cosxamix_amd import forward as F
    c = F.Config(eps=1e-6, **cfg)
    m = F.Modelo(c, tipo=t, semilla=31, tipo_down=tdown, tipo_salida=t)
    names = [x[0] for x in m.tensores()]
    for nm in STAGES[stage]:
        i = names.index(f"blk.0.{nm}.weight")
        write_tensor(m, i, np.zeros(m.tensores()[i][3] // 4, np.float32))
    x, j = R.splitting_vector(c.dim, 7)
    tok, other = 5, 9
    write_tensor(m, names.index("token_embd.weight"), x, byte_offset=tok * c.dim * 4)
    ref = mirror(m)
    # the decode step (one token on an empty cache), then the prefill
    for prompt in ([tok], [other, tok], [tok, other, tok]):
        lg, _ = m.forward(np.array(prompt, np.uint32), m.nueva_cache(8))
        want = ref.forward(np.array(prompt, np.uint32), ref.new_cache(8))
        assert np.array_equal(lg.view(np.uint32), want.view(np.uint32)), (name, stage, prompt)
