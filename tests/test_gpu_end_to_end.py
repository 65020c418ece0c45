"""End to end through the drop-in layer on a tiny random-init Qwen3 decoder
(2 layers, hidden 256, 4 q / 2 kv heads, head_dim 64, RoPE theta 1e6, vocab
4096, weights N(0, 0.02) from a seed), 4 requests with 32-96-token prompts
and 16-row random trees (parents uniform over earlier nodes, depth <= 8),
two verification waves:

  prompts -> prefill (CPU, bf16) -> persistent arena on the GPU
  wave:  pack_block_inputs -> decoder with attn_implementation='specgrove_hip'
         (HIP attention over the arena + the wave's new rows)
         -> lm_head -> hip_tree_rejection verifier -> append_packed_sequence

Checks:
  * every layer's attention output, captured inside the model, equals the
    fp32 oracle (dense packed mask + SDPA over the arena prefixes and the
    layer's new rows) within the attention tolerance, 2e-2 max-abs and 1e-2
    mean-rel;
  * the final hidden states equal the reference wave restated on the CPU in
    bf16 (packed prefixes concatenated into a DynamicCache, the dense additive
    mask, transformers' SDPA) within 1e-2 mean-rel and 0.125 max-abs: two bf16
    runs of the whole model on two devices round differently, and 0.125 is
    4-8 bf16 ulps at the hidden states' magnitude (2-4);
  * the verifier's decisions equal the oracle's on the same logits and
    uniforms bit for bit;
  * the commit moves exactly the kept rows of every layer into the arena.
"""
import copy

import numpy as np
import pytest
import torch

from specgrove_amd import workloads as W

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2      # attention outputs
MEAN_REL = 1e-2
HIDDEN_MAX_ABS = 0.125  # whole-model bf16 hidden states, see the module docstring


class _Layer:
    def __init__(self, keys, values):
        self.keys, self.values = keys, values


class _Cache:
    def __init__(self, layers):
        self.layers = layers

    def get_seq_length(self):
        return int(self.layers[0].keys.shape[-2])


def _tiny_model(transformers):
    cfg = transformers.Qwen3Config(
        hidden_size=256, intermediate_size=768, num_attention_heads=4, num_key_value_heads=2,
        head_dim=64, num_hidden_layers=2, vocab_size=4096, rope_theta=1e6,
        max_position_embeddings=1024, initializer_range=0.02, rms_norm_eps=1e-6,
        tie_word_embeddings=False)
    torch.manual_seed(1234)
    model = transformers.Qwen3ForCausalLM(cfg).eval()
    with torch.no_grad():  # a peaked target distribution, so that drafts get accepted
        model.lm_head.weight.mul_(24.0)
    return model.to(torch.bfloat16)


def test_tiny_qwen3_two_waves_match_the_dense_reference(device, oracle):
    transformers = pytest.importorskip("transformers")
    from transformers import DynamicCache
    from types import SimpleNamespace
    from specgrove_amd import attention, verify
    from specgrove_amd.cache import PersistentRequestCachePool, pack_cache_sequence

    from transformers import AttentionInterface
    captured = {}

    def capture(module, q, k, v, m, **kw):
        out, w = attention.tree_attention_forward(module, q, k, v, m, **kw)
        captured[module.layer_idx] = (q[0].transpose(0, 1).float().cpu(),
                                      k[0].transpose(0, 1).float().cpu(),
                                      v[0].transpose(0, 1).float().cpu(),
                                      out[0].float().cpu(), module.scaling)
        return out, w

    AttentionInterface.register(attention.IMPLEMENTATION, capture)
    cpu_model = _tiny_model(transformers)
    cpu_model.config._attn_implementation = "sdpa"
    gpu_model = copy.deepcopy(cpu_model).to(device)
    gpu_model.config._attn_implementation = attention.IMPLEMENTATION

    rng = np.random.default_rng(11)
    prompts = [rng.integers(0, 4096, size=int(rng.integers(32, 97))) for _ in range(4)]
    caches = []
    with torch.no_grad():
        for p in prompts:
            c = DynamicCache()
            cpu_model.model(input_ids=torch.from_numpy(p[:-1])[None], past_key_values=c,
                            use_cache=True)
            caches.append(_Cache([_Layer(layer.keys.to(device), layer.values.to(device))
                                  for layer in c.layers]))
    pool = PersistentRequestCachePool(caches, capacity=160)
    roots = [int(p[-1]) for p in prompts]

    for wave in range(2):
        parents_list = [W.random_parent_tree(16, rng, max_depth=8) for _ in range(4)]
        tokens_list = [W.random_tokens(p, 4096, rng) for p in parents_list]
        depth_list = [W.depths_of(p) for p in parents_list]
        lengths = list(pool.lengths)
        offsets = list(np.cumsum([0] + lengths[:-1]))

        def run_wave():
            states = [SimpleNamespace(generated=[roots[i]], block_root=0, tree=None,
                                      round_prefix_len=pool.lengths[i],
                                      target_cache=pool.caches[i]) for i in range(4)]
            blocks = [SimpleNamespace(nodes=list(range(16)), parents=parents_list[i],
                                      tokens=tokens_list[i], depths=depth_list[i])
                      for i in range(4)]
            ids, positions, mask, qoff = attention.pack_block_inputs(
                states, blocks, lengths, offsets, sum(lengths), torch.bfloat16, device)
            packed, _, _, total = pack_cache_sequence(pool.caches)
            with torch.no_grad():
                hidden = gpu_model.model(input_ids=ids, position_ids=positions,
                                         attention_mask=mask, past_key_values=packed,
                                         use_cache=True).last_hidden_state
                logits = gpu_model.lm_head(hidden)[0].float()
            return ids, positions, qoff, packed, total, hidden, logits

        # Draft the tree from the target itself, level by level: the children of
        # node p take p's row's top-ranked tokens (row k attends only to its
        # ancestors, so deeper levels do not change shallower rows).
        for depth in range(1, 9):
            *_, logits = run_wave()
            for i in range(4):
                order = torch.argsort(logits[16 * i:16 * i + 16], dim=1, descending=True).cpu()
                used = {}
                for node in range(1, 16):
                    if depth_list[i][node] != depth:
                        continue
                    p = parents_list[i][node]
                    rank = used.get(p, 0)
                    used[p] = rank + 1
                    tokens_list[i][node - 1] = int(order[p, rank])
        ids, positions, qoff, packed, total, hidden, logits = run_wave()
        print(f"wave {wave}: prefixes {lengths}", flush=True)
        with torch.no_grad():

            # Reference wave on the CPU: packed prefix copy + dense mask + SDPA.
            ref_cache = DynamicCache()
            for layer in range(2):
                ref_cache.update(
                    torch.cat([pool.caches[i].layers[layer].keys.cpu() for i in range(4)], 2),
                    torch.cat([pool.caches[i].layers[layer].values.cpu() for i in range(4)], 2),
                    layer)
            dense = torch.from_numpy(oracle.packed_dense_mask(lengths, parents_list))
            ref_hidden = cpu_model.model(
                input_ids=ids.cpu(), position_ids=positions.cpu(),
                attention_mask=dense.to(torch.bfloat16)[None, None], past_key_values=ref_cache,
                use_cache=True).last_hidden_state
        for layer in range(2):
            q, kt, vt, out, scale = captured[layer]
            ks = [pool.caches[i].layers[layer].keys[0].float().cpu() for i in range(4)]
            vs = [pool.caches[i].layers[layer].values[0].float().cpu() for i in range(4)]
            want = oracle.attention_dense(q, ks, vs, kt, vt, parents_list, scale)
            err = (out - want).abs()
            a_max, a_rel = err.max().item(), (err.mean() / want.abs().mean()).item()
            print(f"wave {wave} layer {layer}: attention max_abs {a_max:.3e} "
                  f"mean_rel {a_rel:.3e}", flush=True)
            assert a_max <= MAX_ABS and a_rel <= MEAN_REL
        got = hidden[0].float().cpu()
        ref = ref_hidden[0].float()
        max_abs = (got - ref).abs().max().item()
        mean_rel = ((got - ref).abs().mean() / ref.abs().mean()).item()
        print(f"wave {wave}: hidden max_abs {max_abs:.3e} mean_rel {mean_rel:.3e} "
              f"(|ref| max {ref.abs().max().item():.2f})", flush=True)
        assert max_abs <= HIDDEN_MAX_ABS and mean_rel <= MEAN_REL

        # Verifier vs the oracle on the same logits and uniforms.
        seeds = [1000 * wave + i for i in range(4)]
        results = verify.tree_verify_hip_rejection_batched(
            parents_list, tokens_list, logits,
            generators=[torch.Generator(device).manual_seed(s) for s in seeds])
        depths = [max(W.depths_of(p)) for p in parents_list]
        stride = 2 * (max(depths) + 1)
        uniforms = np.zeros((4, stride), np.float32)
        for i, s in enumerate(seeds):
            g = torch.Generator(device).manual_seed(s)
            uniforms[i, :2 * (depths[i] + 1)] = torch.rand(
                2 * (depths[i] + 1), dtype=torch.float32, device=device, generator=g).cpu().numpy()
        row_offset = np.arange(5, dtype=np.int32) * 16
        parent_flat = np.concatenate([np.asarray(p, np.int32) for p in parents_list])
        token_flat = np.concatenate([np.asarray([-1] + t, np.int32) for t in tokens_list])
        w_nodes, w_len, w_bonus, _, _ = oracle.tree_sample(
            logits.cpu().numpy(), row_offset, parent_flat, token_flat, uniforms, max(depths))
        for i, (nodes, toks, bonus) in enumerate(results):
            assert nodes == w_nodes[i, :w_len[i]].tolist() and bonus == int(w_bonus[i])
            assert toks == [tokens_list[i][n - 1] for n in nodes]
        print(f"wave {wave}: accepted {[len(r[0]) for r in results]}", flush=True)
        if wave == 0:
            assert max(len(r[0]) for r in results) >= 2  # real paths get committed

        # Commit the root + accepted rows of every layer.
        keep = [[0] + nodes for nodes, _, _ in results]
        before = list(pool.lengths)
        pool.append_packed_sequence(packed, pool.caches, total, qoff, keep, device)
        torch.cuda.synchronize()
        assert pool.lengths == [b + len(k) for b, k in zip(before, keep)]
        for layer in range(2):
            for i in range(4):
                got_k = pool.key_storage[layer][:, i * 160 + before[i]:i * 160 + pool.lengths[i]]
                src = packed.layers[layer].keys[0][:, [qoff[i] + r for r in keep[i]]]
                assert torch.equal(got_k, src)
                got_v = pool.value_storage[layer][:, i * 160 + before[i]:i * 160 + pool.lengths[i]]
                assert torch.equal(got_v, packed.layers[layer].values[0][:, [qoff[i] + r
                                                                             for r in keep[i]]])
        roots = [bonus for _, _, bonus in results]
    attention.register()
