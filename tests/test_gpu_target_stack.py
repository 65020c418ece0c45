"""GPU parity of the target decoder stack on the HIP kernels.

* Fused kernels against transformers' own Qwen3 modules on the same bf16
  inputs (the reference runs those modules, engine.py:499-517): the residual
  sum bit-exact; RMSNorm and SiLU * up within 2 bf16 ulps (|a - b| <= 2**-7 *
  |b| + 1e-6: the rsqrt and exp of two libraries may round differently);
  QK-norm + RoPE with transformers' rounding points (each product of the
  rotation, then their sum, rounded to bf16): at least 99.9 % of values
  bit-identical, the rest within 4 bf16 ulps of each rotary pair's magnitude
  (|a - b| <= 2**-6 * sqrt(b_i**2 + b_{i+D/2}**2) + 1e-6; the norm's 1/sqrt
  and sum order and sincos are the device's); the feature gather exact.
* The whole stack on a tiny random-init Qwen3 (2 layers, hidden 256, 4 q / 2
  kv heads, head_dim 64) on one packed wave over the persistent arena, with
  transformers running the same model (HIP attention plug) beside it: against
  an fp32 restatement of the wave on the CPU, the stack's final hidden states
  are at least as close as transformers' bf16 run (mean error within 25 %)
  and within 0.125 everywhere; the new K/V cache rows agree with
  transformers' within 0.125 max-abs and 2e-2 mean-rel; the kept-row features
  equal the stack's own hidden states.
* The decode loop runs on the stack: the logits of its waves match the
  transformers path's within the hidden-state tolerance, and it commits.
"""
import copy

import numpy as np
import pytest
import torch

from specgrove_amd import workloads as W

pytestmark = pytest.mark.gpu

ULP2 = 2.0 ** -7


def _close_bf16(got, want, what):
    got, want = got.float(), want.float()
    err = (got - want).abs()
    bound = want.abs() * ULP2 + 1e-6
    bad = err > bound
    assert not bool(bad.any()), f"{what}: {int(bad.sum())} values beyond 2 ulps, max {err.max()}"


def _close_rotary(got, want, what):
    """Within 4 bf16 ulps of the magnitude of each element's rotary pair."""
    got, want = got.float(), want.float()
    half = want.shape[-1] // 2
    pair = torch.sqrt(want[..., :half] ** 2 + want[..., half:] ** 2)
    bound = torch.cat([pair, pair], dim=-1) * 2.0 ** -6 + 1e-6
    err = (got - want).abs()
    bad = err > bound
    assert not bool(bad.any()), f"{what}: {int(bad.sum())} values beyond the bound, max {err.max()}"


def _tiny_config(transformers):
    return transformers.Qwen3Config(
        hidden_size=256, intermediate_size=768, num_attention_heads=4, num_key_value_heads=2,
        head_dim=64, num_hidden_layers=2, vocab_size=4096, rope_theta=1e6,
        max_position_embeddings=4096, initializer_range=0.02, rms_norm_eps=1e-6,
        tie_word_embeddings=False)


def test_add_rmsnorm_matches_the_transformers_module(device):
    transformers = pytest.importorskip("transformers")
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm
    from specgrove_amd import target
    g = torch.Generator().manual_seed(0)
    for rows, hidden in ((37, 256), (300, 4096), (5, 2560)):
        print(f"add_rmsnorm rows={rows} hidden={hidden}", flush=True)
        x = (torch.randn((rows, hidden), generator=g) * 3).to(torch.bfloat16).to(device)
        res = torch.randn((rows, hidden), generator=g).to(torch.bfloat16).to(device)
        norm = Qwen3RMSNorm(hidden, eps=1e-6).to(device).to(torch.bfloat16)
        with torch.no_grad():
            norm.weight.copy_((1 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16))
            total_ref = x + res
            out_ref = norm(total_ref)
        out, total = target.add_rmsnorm(x, norm.weight, 1e-6, res, want_sum=True)
        assert torch.equal(total, total_ref)
        _close_bf16(out, out_ref, "rmsnorm")
        assert torch.equal(target.add_rmsnorm(x, norm.weight, 1e-6),
                           target.add_rmsnorm(x, norm.weight, 1e-6, None))


@pytest.mark.parametrize("head_dim,hq,hkv", [(64, 4, 2), (128, 32, 8)])
def test_qk_norm_rope_matches_the_transformers_modules(device, head_dim, hq, hkv):
    transformers = pytest.importorskip("transformers")
    from transformers.models.qwen3 import modeling_qwen3 as M
    from specgrove_amd import target
    cfg = transformers.Qwen3Config(hidden_size=hq * head_dim, num_attention_heads=hq,
                                   num_key_value_heads=hkv, head_dim=head_dim, rope_theta=1e6,
                                   max_position_embeddings=65536, rms_norm_eps=1e-6)
    rows = 203
    g = torch.Generator().manual_seed(head_dim)
    qkv = torch.randn((rows, (hq + 2 * hkv) * head_dim), generator=g).to(torch.bfloat16).to(device)
    positions = torch.from_numpy(np.random.default_rng(1).integers(0, 40000, rows)).to(device)
    qn = M.Qwen3RMSNorm(head_dim, eps=1e-6).to(device).to(torch.bfloat16)
    kn = M.Qwen3RMSNorm(head_dim, eps=1e-6).to(device).to(torch.bfloat16)
    with torch.no_grad():
        qn.weight.copy_((1 + 0.2 * torch.randn(head_dim, generator=g)).to(torch.bfloat16))
        kn.weight.copy_((1 + 0.2 * torch.randn(head_dim, generator=g)).to(torch.bfloat16))
        rope = M.Qwen3RotaryEmbedding(cfg).to(device)
        cos, sin = rope(qkv[None], positions[None])
        q_ref = qn(qkv[:, :hq * head_dim].view(1, rows, hq, head_dim)).transpose(1, 2)
        k_ref = kn(qkv[:, hq * head_dim:(hq + hkv) * head_dim].view(1, rows, hkv, head_dim)
                   ).transpose(1, 2)
        q_ref, k_ref = M.apply_rotary_pos_emb(q_ref, k_ref, cos, sin)
    stack_inv = (1.0 / (1e6 ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float()
                                / head_dim))).to(device)
    assert torch.equal(stack_inv, rope.inv_freq.float())
    q, k, v = target.qk_norm_rope(qkv, hq, hkv, head_dim, qn.weight, kn.weight, stack_inv,
                                  positions, 1e-6)
    _close_rotary(q.transpose(0, 1), q_ref[0], "q")
    _close_rotary(k, k_ref[0], "k")
    # The rounding points are transformers' (each product, then the sum): the
    # only differences left come from the norm's 1/sqrt and sum order and
    # from sincos, at most one bf16 ulp away, in a small fraction of values.
    for got, want, what in ((q.transpose(0, 1), q_ref[0], "q"), (k, k_ref[0], "k")):
        same = (got == want).float().mean().item()
        print(f"{what}: {same:.5f} of values bit-identical to transformers", flush=True)
        assert same >= 0.999, (what, same)
    assert torch.equal(v, qkv[:, (hq + hkv) * head_dim:].view(rows, hkv, head_dim).transpose(0, 1))


def test_silu_mul_and_feature_gather(device):
    from specgrove_amd import target
    g = torch.Generator().manual_seed(3)
    gu = (torch.randn((77, 2 * 768), generator=g) * 3).to(torch.bfloat16).to(device)
    want = torch.nn.functional.silu(gu[:, :768]) * gu[:, 768:]
    _close_bf16(target.silu_mul(gu), want, "silu*up")
    layers = [torch.randn((50, 256), generator=g).to(torch.bfloat16).to(device) for _ in range(3)]
    index = torch.tensor([0, 7, 49, 7, 12], dtype=torch.int32, device=device)
    got = target.gather_rows(layers, index)
    assert torch.equal(got, torch.cat([t[index.long()] for t in layers], dim=-1))
    assert int(got.status.item()) == 0
    bad = target.gather_rows(layers, torch.tensor([3, 50], dtype=torch.int32, device=device))
    assert int(bad.status.item()) == -1 and torch.equal(bad[1], torch.zeros_like(bad[1]))


def _tiny_models(transformers, device):
    from specgrove_amd import attention
    from specgrove_amd.target import Qwen3TargetStack
    torch.manual_seed(4321)
    model = transformers.Qwen3ForCausalLM(_tiny_config(transformers)).eval()
    with torch.no_grad():  # a peaked target distribution, so that drafts get accepted
        model.lm_head.weight.mul_(24.0)
    # A bf16 model keeps its rotary inverse frequencies in fp32 (as a model
    # loaded in bf16 has them); Module.to(bfloat16) would round that buffer too.
    rotary = model.model.rotary_emb
    inv_freq = rotary.inv_freq.float().clone()
    model = model.to(torch.bfloat16)
    rotary.inv_freq = inv_freq.clone()
    if hasattr(rotary, "original_inv_freq"):
        rotary.original_inv_freq = inv_freq.clone()
    cpu_model = copy.deepcopy(model)
    gpu_model = model.to(device)
    attention.register()
    gpu_model.config._attn_implementation = attention.IMPLEMENTATION
    return cpu_model, gpu_model, Qwen3TargetStack.from_transformers(gpu_model)


class _Layer:
    def __init__(self, keys, values):
        self.keys, self.values = keys, values


class _Cache:
    def __init__(self, layers):
        self.layers = layers

    def get_seq_length(self):
        return int(self.layers[0].keys.shape[-2])


def _prefill(cpu_model, prompts, device):
    from transformers import DynamicCache
    caches = []
    with torch.no_grad():
        for p in prompts:
            c = DynamicCache()
            cpu_model.model(input_ids=torch.from_numpy(p[:-1])[None], past_key_values=c,
                            use_cache=True)
            caches.append(_Cache([_Layer(layer.keys.to(device), layer.values.to(device))
                                  for layer in c.layers]))
    return caches


def oracle_mask(lengths, parents):
    from oracle import oracle
    return oracle.packed_dense_mask(lengths, parents)


def test_stack_matches_transformers_on_a_packed_wave(device):
    transformers = pytest.importorskip("transformers")
    from types import SimpleNamespace
    from specgrove_amd import attention
    from specgrove_amd.cache import PersistentRequestCachePool, pack_cache_sequence
    cpu_model, gpu_model, stack = _tiny_models(transformers, device)
    rng = np.random.default_rng(12)
    prompts = [rng.integers(0, 4096, size=int(rng.integers(24, 90))) for _ in range(5)]
    pool = PersistentRequestCachePool(_prefill(cpu_model, prompts, device), capacity=160)
    parents = [W.random_parent_tree(int(n), rng, max_depth=6) for n in (16, 9, 1, 24, 12)]
    tokens = [W.random_tokens(p, 4096, rng) for p in parents]
    depths = [W.depths_of(p) for p in parents]
    lengths = list(pool.lengths)
    offsets = list(np.cumsum([0] + lengths[:-1]))
    states = [SimpleNamespace(generated=[int(prompts[i][-1])], block_root=0, tree=None,
                              round_prefix_len=lengths[i], target_cache=pool.caches[i])
              for i in range(5)]
    blocks = [SimpleNamespace(nodes=list(range(len(parents[i]))), parents=parents[i],
                              tokens=tokens[i], depths=depths[i]) for i in range(5)]
    ids, positions, mask, qoff = attention.pack_block_inputs(
        states, blocks, lengths, offsets, sum(lengths), torch.bfloat16, device)
    outs = []
    for runner in (gpu_model.model, stack.model):
        packed, _, _, _ = pack_cache_sequence(pool.caches)
        with torch.no_grad():
            out = runner(input_ids=ids, position_ids=positions, attention_mask=mask,
                         past_key_values=packed, use_cache=True, output_hidden_states=True)
        outs.append((out, packed))
    (ref, ref_cache), (got, got_cache) = outs
    # An fp32 restatement of the wave on the CPU (same bf16 weights and prefix
    # K/V, widened; packed prefixes + the dense mask, as the reference runs
    # it): the stack must be at least as close to it as transformers' own bf16
    # run (within 25 %), and within 0.125 of it everywhere.
    from transformers import DynamicCache
    ref32_model = copy.deepcopy(cpu_model).float()
    ref32_model.config._attn_implementation = "sdpa"
    cache32 = DynamicCache()
    for layer in range(2):
        cache32.update(
            torch.cat([pool.caches[i].layers[layer].keys.float().cpu() for i in range(5)], 2),
            torch.cat([pool.caches[i].layers[layer].values.float().cpu() for i in range(5)], 2),
            layer)
    dense = torch.from_numpy(oracle_mask(lengths, parents))
    with torch.no_grad():
        ref32 = ref32_model.model(input_ids=ids.cpu(), position_ids=positions.cpu(),
                                  attention_mask=dense[None, None], past_key_values=cache32,
                                  use_cache=True).last_hidden_state[0]
    err_got = (got.last_hidden_state[0].float().cpu() - ref32).abs()
    err_hf = (ref.last_hidden_state[0].float().cpu() - ref32).abs()
    print(f"vs fp32 wave: stack mean {err_got.mean():.3e} max {err_got.max():.3e}; "
          f"transformers bf16 mean {err_hf.mean():.3e} max {err_hf.max():.3e}", flush=True)
    assert err_got.mean() <= 1.25 * err_hf.mean() + 1e-4
    assert err_got.max() <= 0.125
    for layer in range(2):
        for name in ("tree_keys", "tree_values"):
            x = getattr(got_cache.layers[layer], name).float()
            y = getattr(ref_cache.layers[layer], name).float()
            assert x.shape == y.shape
            assert (x - y).abs().max().item() <= 0.125
            assert ((x - y).abs().mean() / y.abs().mean()).item() <= 2e-2
    # Draft features of the kept rows: the stack's own hidden states, gathered.
    keep = torch.tensor([qoff[i] + r for i in range(5) for r in (0, len(parents[i]) - 1)],
                        dtype=torch.int32, device=device)
    feats = stack.features(got, [0, 1], keep)
    want = torch.cat([got.hidden_states[1][0][keep.long()], got.hidden_states[2][0][keep.long()]],
                     dim=-1)
    assert torch.equal(feats[0], want)
    assert len(got.hidden_states) == 3 and torch.equal(got.hidden_states[2], got.last_hidden_state)


def test_decode_loop_runs_on_the_stack(device):
    transformers = pytest.importorskip("transformers")
    from specgrove_amd import decode, scheduler
    cpu_model, gpu_model, stack = _tiny_models(transformers, device)
    rng = np.random.default_rng(5)
    prompts = [rng.integers(0, 4096, size=int(rng.integers(24, 60))) for _ in range(3)]

    def run(model):
        caches = _prefill(cpu_model, prompts, device)
        states = [decode.DecodeRequest(request_id=i, generated=[int(p[-1])], target_cache=c,
                                       generator=torch.Generator(device).manual_seed(70 + i))
                  for i, (p, c) in enumerate(zip(prompts, caches))]
        tree_rng = np.random.default_rng(9)

        def propose(state):
            p = W.random_parent_tree(12, tree_rng, max_depth=5)
            return scheduler.DraftTree(p, W.random_tokens(p, 4096, tree_rng), W.depths_of(p))

        records = []
        loop = decode.WaveLoop(model, propose, max_new_tokens=64, capacity=256,
                               on_wave=records.append)
        loop.attach(states)
        for _ in range(3):
            loop.step(states)
        torch.cuda.synchronize()
        return states, records

    ref_states, ref_records = run(gpu_model)
    got_states, got_records = run(stack)
    assert len(got_records) == len(ref_records) >= 1
    # The first wave sees identical inputs: logits within the hidden-state bound.
    a, b = got_records[0].logits.float(), ref_records[0].logits.float()
    rel = ((a - b).abs().mean() / b.abs().mean()).item()
    print(f"decode wave 0 logits mean_rel {rel:.3e}", flush=True)
    assert rel <= 2e-2
    assert all(len(s.generated) > 1 for s in got_states)
