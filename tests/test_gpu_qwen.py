"""The Qwen2-shaped decoder (configuration 5: 24 layers, hidden 896, 14q/2kv heads,
head_dim 64, SwiGLU 4864, vocab 151936, random N(0, 0.02) fp16 weights) served
greedily with continuous batching on the GPU, checked against the CPU restatement
(oracle/model.py): last-position logits of a prompt, and every generated token
teacher-forced (the CPU runs the GPU's own token sequence and predicts each next
token; a different choice is accepted only as a near-tie of the CPU's logits)."""
import numpy as np
import pytest

from kvcache_amd.model import QwenConfig, QwenModel
from oracle import model as M

from _helpers import say

pytestmark = pytest.mark.gpu
NAMES = ("ln1", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "ln2", "wg", "wu", "wd")


def weights(m: QwenModel, cfg: QwenConfig):
    W = {"embed": m.tensor("embed"), "norm": m.tensor("norm")}
    for l in range(cfg.layers):
        for n in NAMES:
            W[f"{n}.{l}"] = m.tensor(n, l)
    return W


@pytest.fixture(scope="module", params=[0, 1], ids=["fused", "op-by-op"])
def small(request):
    cfg = QwenConfig(layers=2, vocab=4096, num_blocks=512, max_batch=8, max_rows=256, seed=11,
                     step_path=request.param)
    m = QwenModel(cfg)
    yield cfg, m, weights(m, cfg)
    m.close()


def test_small_prefill_logits_and_serving(small):
    cfg, m, W = small
    say(f"qwen small: prefill logits, step_path {cfg.step_path}")
    rng = np.random.default_rng(0)
    prompt = rng.integers(0, cfg.vocab, 40)
    tok, lg = m.prefill_logits(prompt)
    ref = M.decoder_logits(W, cfg, prompt)[-1]
    err = np.abs(lg - ref).max()
    print("prefill logits max abs err", err, "logit std", ref.std())
    assert err <= 0.02 * max(1.0, np.abs(ref).max())
    assert tok == int(np.argmax(lg))
    say("qwen small: serving, teacher-forced")
    prompts = [rng.integers(0, cfg.vocab, n) for n in (16, 33, 70, 5, 128, 17, 64, 90, 200, 31)]
    gens = [12, 20, 7, 30, 16, 1, 25, 9, 14, 22]
    out, st = m.serve(prompts, gens)
    assert st["finished"] == len(prompts) and st["tokens"] == sum(gens)
    total_exact = total = 0
    for p, g, o in zip(prompts, gens, out):
        assert len(o) == g
        seq = np.concatenate([p, o[:-1]])
        lc = M.decoder_logits(W, cfg, seq)
        exact, bad = M.teacher_forced_check(lc, len(p), o, margin=0.05)
        assert not bad, bad
        total_exact += exact
        total += g
    print("exact", total_exact, "of", total)
    assert total_exact >= 0.9 * total


def test_graph_replay_matches_eager_steps():
    """The captured decode step (counts and metadata read from device memory)
    replayed step after step, with eager prefills between replays, generates the
    same tokens as the eagerly launched fused step."""
    say("qwen small: graph replay vs eager")
    rng = np.random.default_rng(3)
    prompts = [rng.integers(0, 4096, n) for n in (16, 33, 70, 5, 128, 17, 64, 90, 200, 31, 12, 50)]
    gens = [12, 20, 7, 30, 16, 1, 25, 9, 14, 22, 40, 3]
    outs = {}
    for graph in (0, 1):
        cfg = QwenConfig(layers=2, vocab=4096, num_blocks=512, max_batch=8, max_rows=256, seed=11, graph=graph)
        m = QwenModel(cfg)
        try:
            out, st = m.serve(prompts, gens)
            out2, st2 = m.serve(prompts[:5], gens[:5])  # the graph again, after a reset of the pool
        finally:
            m.close()
        if graph:
            assert st["graph_steps"] == st["steps"] > 0 and st2["graph_steps"] == st2["steps"]
        else:
            assert st["graph_steps"] == 0
        outs[graph] = (out, out2)
    for a, b in zip(outs[0][0] + outs[0][1], outs[1][0] + outs[1][1]):
        np.testing.assert_array_equal(a, b)


def test_config5_shape_prefill_and_generation():
    """The full configuration-5 shape: 24 layers, vocab 151936."""
    say("qwen config 5: prefill + generation")
    cfg = QwenConfig(num_blocks=2048, max_batch=8, max_rows=256, seed=5)
    m = QwenModel(cfg)
    try:
        W = weights(m, cfg)
        rng = np.random.default_rng(1)
        prompts = [rng.integers(0, cfg.vocab, n) for n in (16, 100, 256)]
        gens = [8, 8, 8]
        out, st = m.serve(prompts, gens)
        assert st["finished"] == 3
        total_exact = 0
        for p, o in zip(prompts, out):
            lc = M.decoder_logits(W, cfg, np.concatenate([p, o[:-1]]))
            exact, bad = M.teacher_forced_check(lc, len(p), o, margin=0.05)
            print("exact", exact, "of", len(o), "bad", bad)
            assert not bad, bad
            total_exact += exact
        assert total_exact >= 0.9 * sum(gens)
    finally:
        m.close()
