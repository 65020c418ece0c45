"""The wave loop (specgrove_amd.decode, the decoder's verify-and-commit
sequence on the drop-in path) on a tiny random-init Qwen3 decoder (2 layers,
hidden 256, 4 q / 2 kv heads, head_dim 64, RoPE theta 1e6, vocab 4096,
weights N(0, 0.02) from a seed), 4 requests with 32-96-token prompts.

* Every wave's decisions are checked bit for bit against the oracle sampler
  on the same logits and the same uniforms (redrawn from each request's
  generator state before the wave).
* Persistent arena and non-persistent packing (split after every wave) give
  identical outputs: the attention plans and inputs are the same, so the
  logits are the same bits.
* Continuation blocks and global tiers (the allocator's tier per fresh tree,
  the wave's row budget) run through the same loop.
* The workload as stated (unscaled weights, random 16-node trees with
  uniform draft tokens) runs too.

Drafts come from a CPU copy of the target: a best-first tree of its top
tokens (so that the peaked variant accepts long paths).
"""
import copy

import numpy as np
import pytest
import torch

from specgrove_amd import scheduler as S
from specgrove_amd import workloads as W

pytestmark = pytest.mark.gpu


def _tiny_model(transformers, lm_scale):
    cfg = transformers.Qwen3Config(
        hidden_size=256, intermediate_size=768, num_attention_heads=4, num_key_value_heads=2,
        head_dim=64, num_hidden_layers=2, vocab_size=4096, rope_theta=1e6,
        max_position_embeddings=1024, initializer_range=0.02, rms_norm_eps=1e-6,
        tie_word_embeddings=False)
    torch.manual_seed(1234)
    model = transformers.Qwen3ForCausalLM(cfg).eval()
    if lm_scale != 1.0:
        with torch.no_grad():
            model.lm_head.weight.mul_(lm_scale)
    return model.to(torch.bfloat16)


class _Drafter:
    """Best-first draft trees from a CPU copy of the target: the root's top
    ``width`` tokens, then the top ``width`` under the first child, and so on
    down ``depth`` levels (every node's reach mass from its softmax)."""

    def __init__(self, cpu_model, prompts, width=2, depth=3):
        self.model, self.prompts, self.width, self.depth = cpu_model, prompts, width, depth

    def _next(self, tokens):
        with torch.no_grad():
            logits = self.model(input_ids=torch.tensor(tokens)[None]).logits[0, -1].float()
        return torch.log_softmax(logits, -1)

    def __call__(self, state):
        context = list(self.prompts[state.request_id]) + list(state.generated)
        parents, tokens, depths, masses = [-1], [], [0], [0.0]
        node, path = 0, []
        for level in range(self.depth):
            logp = self._next(context + path)
            top = torch.topk(logp, self.width)
            first = None
            for lp, t in zip(top.values.tolist(), top.indices.tolist()):
                parents.append(node)
                tokens.append(int(t))
                depths.append(level + 1)
                masses.append(masses[node] + lp)
                first = len(parents) - 1 if first is None else first
            node = first
            path.append(tokens[node - 1])
        return S.DraftTree(parents, tokens, depths, masses)


class _RolloutDraft:
    """Per-depth draft probabilities ``q [B, depth, V]`` for DDTree trees: the
    CPU copy's next-token distributions along its own greedy continuation
    (a stand-in for the reference's block draft, which emits one
    distribution per position of the block)."""

    def __init__(self, cpu_model, prompts, depth=4):
        self.model, self.prompts, self.depth = cpu_model, prompts, depth

    def __call__(self, states):
        rows = []
        for s in states:
            context = list(self.prompts[s.request_id]) + list(s.generated)
            qs = []
            for _ in range(self.depth):
                with torch.no_grad():
                    logits = self.model(input_ids=torch.tensor(context)[None]).logits[0, -1]
                qs.append(torch.softmax(logits.float(), -1))
                context.append(int(qs[-1].argmax()))
            rows.append(torch.stack(qs))
        return torch.stack(rows)


class _RandomDrafter:
    """The stated workload's drafts: 16-node trees, parents uniform over
    earlier nodes with depth <= 8, draft tokens uniform over the vocabulary."""

    def __init__(self, seed):
        self.rng = np.random.default_rng(seed)

    def __call__(self, state):
        parents = W.random_parent_tree(16, self.rng, max_depth=8)
        return S.DraftTree(parents, W.random_tokens(parents, 4096, self.rng),
                           W.depths_of(parents))


def _prefill(cpu_model, prompts, device):
    from specgrove_amd.cache import RequestCache
    from transformers import DynamicCache
    caches, anchors = [], []
    with torch.no_grad():
        for p in prompts:
            c = DynamicCache()
            out = cpu_model(input_ids=torch.tensor(p)[None], past_key_values=c, use_cache=True)
            rc = RequestCache()
            for layer_index, layer in enumerate(c.layers):
                rc.update(layer.keys.to(device), layer.values.to(device), layer_index)
            caches.append(rc)
            anchors.append(int(out.logits[0, -1].argmax()))
    return caches, anchors


def _uniforms_from(generator_states, depths, device):
    """The uniforms each request's generator gave the sampler (two per tree
    level), redrawn from its state before the draws."""
    stride = 2 * (max(depths) + 1)
    uniforms = np.zeros((len(depths), stride), np.float32)
    for i, (d, gs) in enumerate(zip(depths, generator_states)):
        g = torch.Generator(device)
        g.set_state(gs)
        uniforms[i, :2 * (d + 1)] = torch.rand(2 * (d + 1), dtype=torch.float32,
                                               device=device, generator=g).cpu().numpy()
    return uniforms


def _wave_checker(oracle, device, waves):
    """on_wave hook: the oracle sampler on the wave's logits with the uniforms
    each request's generator gave the verifier must make the same decisions
    (accepted nodes and tokens, bonus, kept rows)."""
    def check(rec):
        depths = [max(W.depths_of(list(b.parents))) for b in rec.blocks]
        uniforms = _uniforms_from(rec.generator_states, depths, device)
        sizes = [len(b.nodes) for b in rec.blocks]
        row_offset = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
        parent = np.concatenate([np.asarray(b.parents, np.int32) for b in rec.blocks])
        token = np.concatenate([np.asarray([-1] + list(b.tokens), np.int32) for b in rec.blocks])
        nodes, length, bonus, _, _ = oracle.tree_sample(rec.logits.float().cpu().numpy(),
                                                        row_offset, parent, token, uniforms,
                                                        max(depths))
        for i, (got_nodes, got_tokens, got_bonus) in enumerate(rec.results):
            assert list(got_nodes) == nodes[i, :length[i]].tolist()
            assert got_bonus == int(bonus[i])
            assert list(got_tokens) == [rec.blocks[i].tokens[n - 1] for n in got_nodes]
            assert list(rec.keep_rows[i]) == [0] + list(got_nodes)
        waves.append((sizes, [len(r[0]) for r in rec.results]))
        print(f"wave {len(waves)}: rows {sizes} accepted {waves[-1][1]}", flush=True)
    return check


def _decode(setup, device, oracle, *, persistent, drafter, max_new, **kw):
    from specgrove_amd import decode
    gpu_model, cpu_model, prompts = setup
    caches, anchors = _prefill(cpu_model, prompts, device)
    states = [decode.DecodeRequest(i, [anchors[i]], caches[i],
                                   torch.Generator(device).manual_seed(77 + i))
              for i in range(len(prompts))]
    waves = []
    check = _wave_checker(oracle, device, waves)

    capacity = max(len(p) for p in prompts) + max_new + 64
    result = decode.generate_tree_waves(gpu_model, states, drafter, max_new_tokens=max_new,
                                        persistent=persistent, capacity=capacity,
                                        on_wave=check, **kw)
    for s, p in zip(states, prompts):
        assert 1 <= len(s.generated) <= max_new and s.done
        for r in s.rounds:
            assert r["committed_tokens"] <= r["accepted_draft_tokens"] + 1
        if all(r["committed_tokens"] == r["accepted_draft_tokens"] + 1 for r in s.rounds):
            # the cache holds the prompt and every committed token but the newest
            assert s.target_cache.get_seq_length() == len(p) + len(s.generated) - 1
    return result, waves, states


@pytest.fixture(scope="module")
def peaked(device):
    transformers = pytest.importorskip("transformers")
    from specgrove_amd import attention
    attention.register()
    cpu_model = _tiny_model(transformers, 24.0)
    cpu_model.config._attn_implementation = "sdpa"
    gpu_model = copy.deepcopy(cpu_model).to(device)
    gpu_model.config._attn_implementation = attention.IMPLEMENTATION
    rng = np.random.default_rng(11)
    prompts = [rng.integers(0, 4096, size=int(rng.integers(32, 97))).tolist() for _ in range(4)]
    return gpu_model, cpu_model, prompts


def test_persistent_and_split_waves_agree_and_match_the_oracle(peaked, device, oracle):
    drafter = _Drafter(peaked[1], peaked[2])
    a, waves_a, _ = _decode(peaked, device, oracle, persistent=True, drafter=drafter,
                            max_new=24, row_cap=16)
    b, waves_b, _ = _decode(peaked, device, oracle, persistent=False, drafter=drafter,
                            max_new=24, row_cap=16)
    assert a.outputs == b.outputs and waves_a == waves_b
    assert max(n for _, acc in waves_a for n in acc) >= 2   # real paths were committed
    assert a.target_calls < sum(len(o) for o in a.outputs)  # fewer waves than tokens


def test_continuation_blocks_and_stop_ids(peaked, device, oracle):
    """Blocks of 2 rows: an accepted exit edge continues in the same tree (up
    to 3 continuation blocks per round); one request's output stops at a stop
    id drawn from its first round."""
    drafter = _Drafter(peaked[1], peaked[2])
    ref, _, ref_states = _decode(peaked, device, oracle, persistent=True, drafter=drafter,
                                 max_new=12, row_cap=16)
    stop = ref_states[0].generated[3]
    res, _, states = _decode(peaked, device, oracle, persistent=True, drafter=drafter,
                             max_new=12, row_cap=2, max_continuation_blocks=3,
                             stop_ids=[stop])
    assert any(r["continuation_blocks"] > 0 for s in states for r in s.rounds)
    for s in states:  # an output ends at its first stop id, if it has one
        if stop in s.generated:
            assert s.generated.index(stop) == len(s.generated) - 1
    print("stop", stop, "outputs", [len(s.generated) for s in states], flush=True)


def test_global_tiers_respect_the_row_budget(peaked, device, oracle):
    """DDTree trees cut to the allocator's tiers (options 1/3/5 under a 14-row
    wave budget, the reference's option names and contract)."""
    from specgrove_amd import ddtree
    proposer = ddtree.DDTreeProposer(_RolloutDraft(peaked[1], peaked[2]))
    res, waves, states = _decode(peaked, device, oracle, persistent=True, drafter=proposer,
                                 max_new=16, row_cap=2, row_budget=14, tree_budget=5,
                                 global_tree_budget_options=(1, 3, 5),
                                 continuation_ready_threshold=0,
                                 global_tree_fixed_row_equivalent=8.0,
                                 global_tree_criticality_weight=1.0)
    for sizes, _ in waves:
        assert sum(sizes) <= 14 and all(s in (2, 4, 6) for s in sizes)
    assert {b for b, _ in res.effective_tree_budget_counts} <= {1, 3, 5}
    assert res.physical_target_rows == res.useful_target_rows == sum(
        sum(sizes) for sizes, _ in waves)


def test_ddtree_trees_with_occupancy_controls(peaked, device, oracle):
    """DDTree trees from per-depth draft probabilities (the best-first builder
    of tree.py:148-212), 4-node trees while more than two requests are
    active and 12-node trees for the one most behind after that, blocks of 5
    rows widened to 13 at low occupancy; persistent and non-persistent waves
    agree and every wave matches the oracle."""
    from specgrove_amd import ddtree
    proposer = ddtree.DDTreeProposer(_RolloutDraft(peaked[1], peaked[2]))
    kw = dict(max_new=20, row_cap=5, row_budget=64, tree_budget=12, proposal_tree_budget=4,
              low_occupancy_tree_budget=12, low_occupancy_tree_threshold=2,
              low_occupancy_expansion_slots=1, low_occupancy_row_cap=13,
              low_occupancy_threshold=2)
    a, waves_a, _ = _decode(peaked, device, oracle, persistent=True, drafter=proposer, **kw)
    b, waves_b, _ = _decode(peaked, device, oracle, persistent=False, drafter=proposer, **kw)
    assert a.outputs == b.outputs and waves_a == waves_b
    budgets = dict(a.effective_tree_budget_counts)
    caps = dict(a.effective_row_cap_counts)
    assert set(budgets) <= {4, 12} and budgets[4] >= 4
    assert set(caps) <= {5, 13} and caps[5] >= 1
    assert sum(caps.values()) == a.physical_target_calls
    print("tree budgets", budgets, "row caps", caps, "gated", a.gated_continuations, flush=True)


def test_stated_tiny_workload(device, oracle):
    """Unscaled N(0, 0.02) weights, random 16-node trees, uniform draft tokens
    over the 4096-token vocabulary, rows packed to 64."""
    transformers = pytest.importorskip("transformers")
    from specgrove_amd import attention
    attention.register()
    cpu_model = _tiny_model(transformers, 1.0)
    cpu_model.config._attn_implementation = "sdpa"
    gpu_model = copy.deepcopy(cpu_model).to(device)
    gpu_model.config._attn_implementation = attention.IMPLEMENTATION
    rng = np.random.default_rng(12)
    prompts = [rng.integers(0, 4096, size=int(rng.integers(32, 97))).tolist() for _ in range(4)]
    res, waves, _ = _decode((gpu_model, cpu_model, prompts), device, oracle, persistent=True,
                            drafter=_RandomDrafter(13), max_new=4, row_cap=16, row_budget=64)
    assert waves[0][0] == [16, 16, 16, 16] and all(sum(sizes) <= 64 for sizes, _ in waves)


def test_open_loop_serving(peaked, device, oracle):
    """Six requests arriving over 40 ms, at most three active, one prompt of
    300 tokens (two prefill chunks).  Newcomers are prefilled in packed waves
    through the HIP attention (prompts as causal chains) and their first
    token drawn by the HIP sampler; the non-persistent wave loop runs between
    admissions.  Checked: every wave's decisions and every first-token draw
    against the oracle, the prefilled K/V against the CPU model's prefill,
    the admission rule at every boundary, and the latency accounting."""
    from specgrove_amd import decode, serving
    from tests.test_serving import check_admissions
    gpu_model, cpu_model, prompts = peaked
    rng = np.random.default_rng(21)
    prompts = prompts + [prompts[0], rng.integers(0, 4096, size=300).tolist()]
    drafter = _Drafter(cpu_model, prompts)
    states = [decode.DecodeRequest(i, [], None, torch.Generator(device).manual_seed(90 + i))
              for i in range(len(prompts))]
    draws = []

    def on_chunk(ids, rows, logits, gen_states):
        uniforms = _uniforms_from(gen_states, [0] * len(ids), device)
        n = len(ids)
        _, _, bonus, _, _ = oracle.tree_sample(
            logits.float().cpu().numpy(), np.arange(n + 1, dtype=np.int32),
            np.full(n, -1, np.int32), np.full(n, -1, np.int32), uniforms, 0)
        draws.append((tuple(ids), tuple(int(b) for b in bonus)))

    prefill = serving.PackedPrefill(gpu_model, prompts, on_chunk=on_chunk)
    waves = []
    arrivals = [0.0, 0.0, 0.005, 0.01, 0.02, 0.04]
    res = serving.serve_open_loop(gpu_model, states, arrivals, drafter, prefill,
                                  max_active_requests=3, max_new_tokens=10, row_cap=16,
                                  on_wave=_wave_checker(oracle, device, waves))
    assert res.max_concurrent <= 3 and len(waves) == res.target_calls
    check_admissions(res, arrivals, 3)
    first = {k: s.generated[0] for k, s in enumerate(states)}
    assert sorted(k for ids, _ in draws for k in ids) == list(range(len(prompts)))
    for ids, bonus in draws:
        assert [first[k] for k in ids] == list(bonus)
    for s, m in zip(states, res.request_metrics):
        assert s.done and 1 <= len(s.generated) <= 10 and m["output_tokens"] == len(s.generated)
        assert 0 <= m["queue_ms"] <= m["ttft_ms"] <= m["e2e_ms"]
        assert m["arrival_ms"] <= m["admitted_ms"]
    # the packed prefill's K/V against the CPU model's own prefill of each prompt
    probe = [decode.DecodeRequest(k, [], None, torch.Generator(device).manual_seed(5))
             for k in (0, 5)]
    serving.PackedPrefill(gpu_model, prompts)(probe)
    ref, _ = _prefill(cpu_model, [prompts[0], prompts[5]], device)
    for s, r in zip(probe, ref):
        assert s.target_cache.get_seq_length() == r.get_seq_length() == len(prompts[s.request_id])
        for layer, (a, b) in enumerate(zip(s.target_cache.layers, r.layers)):
            for x, y in ((a.keys, b.keys), (a.values, b.values)):
                x, y = x.float(), y.float()
                rel = ((x - y).abs().mean() / y.abs().mean()).item()
                assert rel <= 1e-2, (s.request_id, layer, rel)
    print("metrics", [(round(m["ttft_ms"], 1), round(m["tpot_ms"], 2))
                      for m in res.request_metrics], "admissions",
          [a["admitted"] for a in res.admissions], flush=True)
