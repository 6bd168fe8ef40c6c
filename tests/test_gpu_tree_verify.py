"""qwn_hip_decoder_verify_tree / qwn_hip_decoder_commit_path: the target-side
forward of a speculative draft TREE (c/qwanto_jetspec.h:17-33), against the
oracle decoder stepping each node's root-to-node path after the same prefix.

In the tree forward node i sits at cache slot P + i but is rotated for
position P + depth(i), and attends to the prefix, its ancestors and itself
only (qwn_jetspec_build_tree_mask, c/qwanto_jetspec.c:33-49): exactly the
context a chain forward of its path gives it.  So the logits after node i
must be the oracle's after prefix + path(i), within the oracle's rounding
envelope on that path (parity.within_envelope); a node that saw a sibling,
or was rotated for its slot instead of its depth, is off by orders of
magnitude more.  After commit_path the accepted path's K/V sit in slots
P .. P + len - 1: the next step matches the oracle after prefix + path, and
the cache matches a decoder that prefilled prefix + path (one int8 step at
rounding boundaries, as the prefill test allows)."""
import numpy as np
import pytest

from parity import ENV_K, oracle_envelope, step_errors, within_envelope
from qwanto_amd import abi, synth

pytestmark = pytest.mark.gpu

SMALL = dict(hidden=256, intermediate=512, layers=2, heads=4, kv_heads=2, head_dim=64, vocab=1000,
             max_ctx=128, rope_theta=1e6, rms_eps=1e-6)
QWEN2_LIKE = dict(hidden=768, intermediate=1024, layers=3, heads=6, kv_heads=1, head_dim=128, vocab=4096,
                  max_ctx=128, rope_theta=1e6, rms_eps=1e-6)
# past one split: the MFMA split attention with the tree mask
LONG_CTX = dict(SMALL, max_ctx=1500)
# one split, past the fused decode attention's first 256-token chunks
MID_CTX = dict(SMALL, max_ctx=640)
ENV_SEEDS = tuple(range(1, 9))


def with_norms(rng, model):
    D = model["cfg"]["hidden"]
    for layer in model["layers"]:
        layer["input_norm"] = (1.0 + 0.2 * rng.standard_normal(D)).astype(np.float32)
        layer["post_norm"] = (1.0 + 0.2 * rng.standard_normal(D)).astype(np.float32)
    model["final_norm"] = (1.0 + 0.2 * rng.standard_normal(D)).astype(np.float32)
    return model


def random_tree(rng, level_sizes, vocab):
    """Nodes level by level (breadth first, so parents come first): level 0
    are roots (-1), every node of level k has a random parent in level k-1."""
    parents, levels = [], []
    for k, n in enumerate(level_sizes):
        prev = levels[-1] if levels else []
        cur = []
        for _ in range(n):
            parents.append(-1 if k == 0 else int(prev[rng.integers(len(prev))]))
            cur.append(len(parents) - 1)
        levels.append(cur)
    tokens = rng.integers(0, vocab, len(parents)).astype(np.int32)
    return tokens, np.array(parents, dtype=np.int32)


def path_to(parents, i):
    p = []
    while i >= 0:
        p.append(int(i))
        i = int(parents[i])
    return p[::-1]


@pytest.mark.parametrize("cfg,dtype,P,levels,head", [
    (SMALL, "q4_0", 20, (3, 8, 14, 15), None), (QWEN2_LIKE, "hvsq2", 12, (3, 8, 14, 15), None),
    (QWEN2_LIKE, "q4_0", 7, (3, 8, 14, 15), None), (LONG_CTX, "hvsq2", 300, (3, 8, 14, 15), None),
    # an untied BF16 head (three pieces per token) through the 32-token head launches
    (QWEN2_LIKE, "q4_0", 9, (2, 4, 6, 8, 10, 10, 12, 12), "bf16"),
    # 64 nodes (one block of four 16-token MFMA groups), depth 8: the reference's limits (c/qwanto_jetspec.h:17-18)
    (SMALL, "hvsq2", 9, (2, 4, 6, 8, 10, 10, 12, 12), None),
    (LONG_CTX, "q4_0", 600, (1, 3, 6, 10, 14, 14, 16), None),
    # nodes straddling the 256- and 512-token chunk boundaries
    (MID_CTX, "q4_0", 240, (3, 8, 14, 15), None), (MID_CTX, "hvsq2", 500, (2, 4, 6, 8, 10, 10, 12, 12), None)])
def test_tree_verify_matches_oracle_paths(gpu_ctx, oracle_lib, cfg, dtype, P, levels, head):
    rng = np.random.default_rng(1300 + P + sum(levels))
    model = with_norms(rng, synth.decoder_model(rng, cfg, dtype, lm_head=head))
    prompt = synth.prompt_tokens(rng, cfg["vocab"], P)
    tokens, parents = random_tree(rng, levels, cfg["vocab"])
    n = tokens.size
    assert n <= 64
    # oracle: prefix + path for every leaf; each node's logits from a path through it
    children = {i: [j for j in range(n) if parents[j] == i] for i in range(n)}
    leaves = [i for i in range(n) if not children[i]]
    ref_logits, env_cols = {}, {}
    for leaf in leaves:
        path = path_to(parents, leaf)
        d = oracle_lib.decoder(model)
        steps = [d.forward(int(t)) for t in list(prompt) + [int(tokens[i]) for i in path]]
        d.close()
        inputs = list(prompt) + [int(tokens[i]) for i in path]
        env = oracle_envelope(oracle_lib, model, inputs, steps, seeds=ENV_SEEDS)
        for k, node in enumerate(path):
            if node not in ref_logits:
                ref_logits[node] = steps[P + k]
                env_cols[node] = env[:, P + k]
    dec = abi.ResidentDecoder(gpu_ctx, model)
    dec2 = abi.ResidentDecoder(gpu_ctx, model)
    try:
        _, _ = dec.prefill(prompt, logits=False)
        logits, ids = dec.verify_tree(tokens, parents)
        assert ids.tolist() == [int(np.argmax(r)) for r in logits]
        errs = step_errors([logits[i] for i in range(n)], [ref_logits[i] for i in range(n)])
        env = np.stack([env_cols[i] for i in range(n)], axis=1)
        ok, msg = within_envelope(errs, env)
        assert ok, f"tree nodes vs oracle paths: {msg}"
        # commit the deepest path, then one more step
        leaf = max(leaves, key=lambda i: len(path_to(parents, i)))
        path = path_to(parents, leaf)
        with pytest.raises(abi.AbiError):  # not a root-to-node chain
            dec.commit_path(path[1:])
        dec.commit_path(path)
        nxt = int(rng.integers(cfg["vocab"]))
        after, _ = dec.forward(nxt)
        L = len(path)
        committed = [dec.kv_read(l, P, L) for l in range(cfg["layers"])]
        # a decoder that prefilled prefix + path: the same cache contents
        dec2.prefill(np.concatenate([prompt, tokens[path]]), logits=False)
        chained = [dec2.kv_read(l, P, L) for l in range(cfg["layers"])]
    finally:
        dec.close()
        dec2.close()
    inputs = list(prompt) + [int(tokens[i]) for i in path] + [nxt]
    d = oracle_lib.decoder(model)
    steps = [d.forward(int(t)) for t in inputs]
    d.close()
    env = oracle_envelope(oracle_lib, model, inputs, steps, seeds=ENV_SEEDS)
    ok, msg = within_envelope(step_errors([after], [steps[-1]]), env[:, -1:])
    assert ok, f"step after commit vs oracle: {msg}"
    for l, (a, b) in enumerate(zip(committed, chained)):
        for name, x, y in (("keys", a[0], b[0]), ("values", a[1], b[1])):
            dd = np.abs(x.astype(np.int32) - y.astype(np.int32))
            frac = float(np.mean(dd > 0))
            limit = 0.02 if l == 0 else 0.05
            assert frac <= limit and (l > 0 or dd.max() <= 1), \
                f"layer {l} {name}: {frac:.3%} of committed entries differ from a chain prefill (by up to {dd.max()})"


def test_tree_contract(gpu_ctx):
    """Refusals: a parent that is not an earlier node, more than 64 nodes, a
    commit with no verified tree, a commit after another call dropped the
    tree; a chain tree (each node the child of the previous) gives the
    logits of the block verify of the same tokens."""
    rng = np.random.default_rng(5)
    model = with_norms(rng, synth.decoder_model(rng, SMALL, "q4_0"))
    dec = abi.ResidentDecoder(gpu_ctx, model)
    try:
        dec.prefill(synth.prompt_tokens(rng, SMALL["vocab"], 8), logits=False)
        toks = synth.prompt_tokens(rng, SMALL["vocab"], 6)
        with pytest.raises(abi.AbiError):
            dec.verify_tree(toks, [-1, 0, 2, 1, 1, 1])          # parent 2 of node 2: not earlier
        with pytest.raises(abi.AbiError):
            dec.verify_tree(np.zeros(65, np.int32), [-1] * 65)   # more than 64 nodes
        with pytest.raises(abi.AbiError):
            dec.commit_path([0])                                 # nothing verified
        chain, ids_c = dec.verify_tree(toks, [-1, 0, 1, 2, 3, 4])
        block, ids_b = dec.verify(toks)                          # the same tokens as a chain block
        ok, msg = within_envelope(step_errors(list(chain), list(block)), np.full((1, 6), 1e-6), k=1.0)
        assert ok, f"chain tree vs verify block: {msg}"
        with pytest.raises(abi.AbiError):
            dec.commit_path([0, 1])                              # verify() dropped the tree
    finally:
        dec.close()
