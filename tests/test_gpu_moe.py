"""MoE edge cases of the reference's tests (tests/test_moe.py:147-157, 370-406), through the engine ABI on
the GPU, on both MoE paths: the prompt's prefill chunk (16 tokens x top-2 = 32 routed rows: the router,
sort and grouped GEMMs on the device; SARDYNE_NO_GROUPED_MOE=1 groups the experts on the host instead)
and one-token decode steps (device router, grouped matvec over the routed experts, replayed from the
recorded decode graph).

  - unused experts poisoned with NaN scales change no bit of the logits: only routed experts are read;
  - identical experts equal the dense MLP of the same weights (the renormalised weights sum to 1);
  - an all-zero router gives equal probabilities, and ties pick the lowest expert indices (poisoning
    every expert from k upwards changes nothing, and the logits equal the reference engine's).
"""
import dataclasses

import numpy as np
import pytest

import oracle as O
from conftest import engine_env
from moe_cases import MOE, PROMPT, STEPS, poison_experts, used_experts
from sardyne_amd.engine import LoadedModel
from sardyne_amd.gguf_synth import write_model

pytestmark = pytest.mark.gpu


def run(path, n_batch=16, mode="exact", **switches):
    """Prompt logits, then one-token steps' logits (stacked), with the one-token attention `mode`
    (SARDYNE_ATTENTION: exact, chunked or split) and the environment switches given, set while the
    model loads and the context is made."""
    with engine_env(SARDYNE_ATTENTION=mode, **switches):
        model = LoadedModel(path)
        s = model.session(max_seq=48, n_batch=n_batch)
    return np.stack([s.feed(PROMPT)] + [s.step(t) for t in STEPS])


@pytest.mark.parametrize("switch", ["SARDYNE_UPLOAD_SYNC", "SARDYNE_NO_GROUPED_MOE", "SARDYNE_GEMM_COPY_MB"])
def test_load_and_prefill_switches_keep_the_bits(tmp_path, switch):
    """The synchronous per-tensor upload, the host-grouped MoE prefill and a load without the GEMM's
    tiled weight copies give the default run's logits bit for bit."""
    p = write_model(tmp_path / "m.gguf", MOE, seed=3)
    base = run(p)
    got = run(p, **{switch: "0" if switch == "SARDYNE_GEMM_COPY_MB" else "1"})
    assert np.all(np.isfinite(base))
    assert np.array_equal(base.view(np.uint32), got.view(np.uint32))


def test_unused_experts_poisoned_with_nan_change_nothing(tmp_path):
    clean_p = write_model(tmp_path / "clean.gguf", MOE, seed=3)
    used = used_experts(clean_p)
    unused = [sorted(set(range(MOE.n_expert)) - u) for u in used]
    assert all(len(u) >= MOE.n_expert // 2 for u in unused)
    dirty_p = write_model(tmp_path / "dirty.gguf", MOE, seed=3)
    poison_experts(dirty_p, unused)
    clean, dirty = run(clean_p), run(dirty_p)
    assert np.all(np.isfinite(clean))
    assert np.array_equal(clean.view(np.uint32), dirty.view(np.uint32))
    # the split attentions read only routed experts too
    for mode in ("chunked", "split"):
        assert np.array_equal(run(clean_p, mode=mode).view(np.uint32), run(dirty_p, mode=mode).view(np.uint32))
    # a poisoned expert that is routed does reach the logits (the poisoning is effective). The Q8_K
    # activation quantiser of the next matvec takes its maximum over |x| with ordered comparisons, so
    # NaN rows quantise to zero blocks and the logits stay finite: the reference does exactly that,
    # and the GPU must give its bits
    hit_p = write_model(tmp_path / "hit.gguf", MOE, seed=3)
    poison_experts(hit_p, [sorted(used[0])[:1], []])
    hit = run(hit_p)
    assert np.any(hit.view(np.uint32) != clean.view(np.uint32))
    if O.ref_available():
        ref = O.RefEngine(hit_p, 48, n_batch=16)
        exp = np.stack([ref.eval(PROMPT)] + [ref.eval([t]) for t in STEPS])
        assert np.array_equal(hit.view(np.uint32), exp.view(np.uint32))


@pytest.mark.parametrize("n_expert,n_used", [(1, 1), (5, 5), (8, 3)], ids=["one", "all", "topk"])
def test_identical_experts_equal_dense(tmp_path, n_expert, n_used):
    moe = dataclasses.replace(MOE, n_expert=n_expert, n_expert_used=n_used, same_experts=True)
    dense = dataclasses.replace(MOE, arch="qwen3", ffn_dim=MOE.ffn_exp_dim, n_expert=0, n_expert_used=0,
                                ffn_exp_dim=0)
    got = run(write_model(tmp_path / "moe.gguf", moe, seed=4))
    exp = run(write_model(tmp_path / "dense.gguf", dense, seed=4))
    # the weights sum to 1 up to rounding: the reference test's scale-relative tolerance
    np.testing.assert_allclose(got, exp, atol=1e-4 * max(1.0, float(np.abs(exp).max())), rtol=0)
    assert np.array_equal(got.argmax(-1), exp.argmax(-1))


def test_zero_router_picks_the_lowest_experts(tmp_path):
    spec = dataclasses.replace(MOE, n_expert=16, n_expert_used=4, router_std=0.0)
    clean_p = write_model(tmp_path / "zero.gguf", spec, seed=5)
    clean = run(clean_p)
    ref = O.RefEngine(clean_p, 48, n_batch=16) if O.ref_available() else None
    if ref is not None:
        exp = np.stack([ref.eval(PROMPT)] + [ref.eval([t]) for t in STEPS])
        assert np.array_equal(clean.view(np.uint32), exp.view(np.uint32))
    high_p = write_model(tmp_path / "high.gguf", spec, seed=5)
    poison_experts(high_p, [range(4, 16)] * spec.n_layer)
    high = run(high_p)
    assert np.array_equal(clean.view(np.uint32), high.view(np.uint32))
