"""Residency plan with a GPU tier (qwn_hip_ext_plan_residency) against the
reference's qwn_plan_residency (c/qwanto_native.c:379-435) built in place
(oracle/_ref), on .qwn files written by qwanto_amd/qwn_file.py, plus a
hand-checked case.  Host code only: no GPU is touched with an explicit
budget."""
import os

import numpy as np
import pytest

from qwanto_amd import abi, qwn_file


def model_tensors(rng, layers=3, experts=2):
    """Tensor names of every priority class, F32 payloads of varied sizes
    (more than the inline index holds, so overflow descriptors count too)."""
    names = ["model.embed_tokens.weight", "lm_head.weight", "model.norm.weight", "model.rotary.inv_freq"]
    for l in range(layers):
        p = f"model.layers.{l}."
        names += [p + "input_layernorm.weight", p + "post_attention_layernorm.weight"]
        names += [p + f"self_attn.{x}_proj.weight" for x in "qkvo"]
        names += [p + f"mlp.{x}_proj.weight" for x in ("gate", "up", "down")]
        names += [p + "block_sparse_moe.gate.weight"]
        names += [p + f"mlp.experts.{e}.{x}_proj.weight" for e in range(experts) for x in ("gate", "up")]
    out = []
    for n in names:
        numel = int(rng.integers(1, 600)) * (16 if rng.random() < 0.5 else 1)
        out.append((n, qwn_file.DT_F32, (numel,), rng.standard_normal(numel).astype(np.float32)))
    # equal sizes within a priority class exercise the index tie-break
    out.append(("model.layers.0.self_attn.extra_attn.weight", qwn_file.DT_F32, (16,), np.zeros(16, np.float32)))
    out.append(("model.layers.1.self_attn.extra_attn.weight", qwn_file.DT_F32, (16,), np.zeros(16, np.float32)))
    return out


def our_plan(hip, path, gpu, ram):
    f = qwn_file.QwnFile(path)
    try:
        names = list(f.tensors)
        offs = [f.tensors[n]["offset"] for n in names]
        sizes = [f.tensors[n]["size"] for n in names]
    finally:
        f.close()
    items, totals = abi.plan_residency(hip, names, offs, sizes, gpu, ram)
    rows = [(p.name_hash, p.byte_offset, p.byte_size, p.tensor_index, p.tier, p.priority) for p in items]
    return rows, totals, names, sizes


@pytest.fixture(scope="module")
def hip():
    return abi.load()


def test_plan_matches_reference(hip, ref_lib, tmp_path):
    rng = np.random.default_rng(12)
    path = str(tmp_path / "plan.qwn")
    tensors = model_tensors(rng)
    assert len(tensors) > qwn_file.INLINE_MAX
    qwn_file.write_qwn(path, tensors)
    total = None
    for gpu, ram in [(0, 0), (1 << 40, 0), (4096, 0), (20000, 5000), (50000, 1 << 40), (0, 30000),
                     (123457, 77777)]:
        ours, tot, names, sizes = our_plan(hip, path, gpu, ram)
        ref, rtot = ref_lib.plan_residency(path, gpu, ram, len(names))
        assert ours == ref, f"budgets {gpu}/{ram}: plans differ"
        assert tot == rtot
        total = sum(sizes)
        assert sum(tot) == total


def test_plan_hand_checked(hip):
    """Order: priority (embed 255, norm 245, attention 230, dense gate 210,
    other 160, expert 80), then size, then index; GPU fills first, then
    RAM; a tensor that fits neither stays file-backed even when a later,
    smaller one fits."""
    names = ["x.experts.0.w", "model.embed_tokens.weight", "model.layers.0.mlp.gate_proj.weight",
             "model.norm.weight", "model.layers.0.self_attn.q_proj.weight", "misc.table", "misc.small"]
    sizes = [60, 100, 50, 4, 30, 45, 5]
    items, totals = abi.plan_residency(hip, names, [10 * i for i in range(7)], sizes, 150, 50)
    order = [p.tensor_index for p in items]
    assert order == [1, 3, 4, 2, 6, 5, 0]
    tiers = {p.tensor_index: p.tier for p in items}
    # 100 + 4 + 30 on the GPU (gate 50 would pass 150), gate 50 -> RAM,
    # small 5 -> GPU (139), table 45 -> RAM? 50 + 45 > 50 -> file, expert 60 -> file
    assert tiers == {1: abi.TIER_GPU, 3: abi.TIER_GPU, 4: abi.TIER_GPU, 2: abi.TIER_RAM, 6: abi.TIER_GPU,
                     5: abi.TIER_FILE, 0: abi.TIER_FILE}
    assert totals == (139, 50, 105)
    assert [p.priority for p in items] == [255, 245, 230, 210, 160, 160, 80]
    assert items[0].name_hash == qwn_file.fnv1a64("model.embed_tokens.weight")


def test_plan_auto_budget_needs_context(hip):
    with pytest.raises(abi.AbiError):
        abi.plan_residency(hip, ["a"], [0], [1], abi.GPU_BUDGET_AUTO, 0)
