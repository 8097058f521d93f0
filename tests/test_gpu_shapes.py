"""End-to-end parity on model shapes other than the golden ones: head_dim 128
and 32, query heads per KV head 1, 3 and 8, FFN widths and vocabularies that
are not multiples of the tile sizes.  The GPU path (decode, GEMM prefill,
batched decode) is compared with the CPU oracle, which the reference build
pins bit for bit (tests/test_oracle.py): greedy ids identical, logits within
max |gpu - oracle| / max |oracle| <= 2e-3.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_err

pytestmark = pytest.mark.gpu
TOL = 2e-3

SHAPES = {
    # name: config overrides (random N(0, 0.02) fp16-representable weights, seed 7)
    "d128_r1": dict(hidden_size=256, num_hidden_layers=2, num_attention_heads=2, num_key_value_heads=2, head_dim=128,
                    intermediate_size=768, vocab_size=1000),
    "d64_r8": dict(hidden_size=512, num_hidden_layers=2, num_attention_heads=8, num_key_value_heads=1, head_dim=64,
                   intermediate_size=1408, vocab_size=777),
    "d64_r3": dict(hidden_size=384, num_hidden_layers=3, num_attention_heads=6, num_key_value_heads=2, head_dim=64,
                   intermediate_size=1000, vocab_size=4097),
    "d32_r2": dict(hidden_size=128, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2, head_dim=32,
                   intermediate_size=344, vocab_size=300),
}
BASE = dict(max_position_embeddings=4096, rms_norm_eps=1e-5, rope_theta=1e6, tie_word_embeddings=1)


@pytest.fixture(scope="module", params=sorted(SHAPES))
def shape_model(request, gpu, oracle, tmp_path_factory):
    name = request.param
    print(f"[case] shape {name}", flush=True)
    cfg = gpu.make_config(**{**BASE, **SHAPES[name]})
    d = tmp_path_factory.mktemp(name)
    gpu.write_synthetic_model(d, cfg, 7, 0.02, True)
    return name, d, gpu.Model.load(d), oracle.OracleModel(d)


def test_decode_matches_oracle(gpu, shape_model):
    name, _, m, om = shape_model
    V = om.vocab
    rng = np.random.default_rng(len(name))
    prompt = [int(t) for t in rng.integers(0, V, 11)]
    ref_tokens = om.generate(prompt, 24)
    assert m.generate(prompt, 24) == ref_tokens, name
    # per-step logits through forward_token on both sides
    st, ost = m.make_state(64), om.new_state()
    for i, tok in enumerate(prompt + ref_tokens[:-1]):
        lg, ref = st.forward_token(tok), ost.forward_token(tok)
        if i in (0, 10, 20, len(prompt) + len(ref_tokens) - 2):
            assert rel_err(lg, ref) < TOL, (name, i)
            assert int(np.argmax(lg)) == int(np.argmax(ref))


def test_gemm_prefill_and_batch_match_oracle(gpu, shape_model, monkeypatch):
    # 150-token prompt through the chunked GEMM prefill (chunk 64: three
    # chunks), then decode; and the same prompts in a batch of three
    name, _, m, om = shape_model
    V = om.vocab
    rng = np.random.default_rng(100 + len(name))
    prompts = [[int(t) for t in rng.integers(0, V, n)] for n in (150, 37, 90)]
    monkeypatch.setenv("MMR_PREFILL_CHUNK", "64")
    st = m.make_state(200)
    monkeypatch.delenv("MMR_PREFILL_CHUNK")
    ref0 = om.generate(prompts[0], 12)
    st.enqueue_prefill(prompts[0])
    st.enqueue_decode(11)
    st.synchronize()
    assert st.read_sequence(150, 12).tolist()[: len(ref0)] == ref0, name  # the oracle stops after EOS
    bs = m.make_batch_state(3, 200, gpu.KV_F32)
    bs.prefill(prompts)
    bs.decode(12)
    bs.synchronize()
    for b, p in enumerate(prompts):
        n_new = 150 + 12 - len(p) + 1
        ref = om.generate(p, n_new)
        assert bs.read_sequence(b, len(p), n_new).tolist()[: len(ref)] == ref, (name, b)
