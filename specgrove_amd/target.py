"""The target model's decoder stack for packed verification waves, on the
HIP kernels: a Qwen3 causal LM (embedding, decoder layers, final norm, LM head)
whose attention is the request-isolated tree attention over the persistent
arena (or a non-persistent wave's packed prefixes), whose elementwise stages
are the fused kernels of ``csrc/layer_ops.hip`` and whose projections are
library GEMMs (hipBLASLt through ``torch.matmul``).

It replaces the transformers decoder that the reference runs per wave
(``Engine.target_hidden_forward``, engine.py:499-517; transformers' Qwen3
modules) and the draft-feature gather of the kept rows
(continuous_tree_block_decode.py:2144-2158, ``engine.features`` :446):

* ``Qwen3TargetStack.from_transformers(model)`` takes the weights of a
  ``Qwen3ForCausalLM`` (q/k/v and gate/up merged into one matrix each);
* ``stack.model(input_ids=, position_ids=, attention_mask=, past_key_values=,
  use_cache=True)`` has the call shape of ``model.model(...)`` in the decode
  loop: ``attention_mask`` is the wave's ``PackedTreeMask`` (as
  ``{"full_attention": mask}``), ``past_key_values`` its ``TreeVerifyCache``,
  which receives every layer's new K/V rows;
* ``stack.get_output_embeddings()`` is the LM head (``lm_head.weight`` for
  ``sg_lm_head``);
* ``stack.features(output, keep_index)`` gathers the kept rows of the
  draft's target layers in one launch.

Per layer: add+RMSNorm -> [q|k|v] projection -> QK-norm + RoPE (writing q and
the cache rows) -> tree attention -> o projection -> add+RMSNorm -> [gate|up]
projection -> SiLU * up -> down projection; the residual add of each block is
folded into the next add+RMSNorm.  Hidden states follow the reference's
transformers convention (``hidden_states[i + 1]`` is layer i's output for
i < L - 1 and the final normed output for i = L - 1).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from types import SimpleNamespace
from typing import Sequence

import torch

from . import _lib, attention, ops


def _stream():
    return ctypes.c_void_p(ops._stream_handle())


def add_rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float,
                residual: torch.Tensor | None = None, want_sum: bool = False):
    """RMSNorm(x + residual) and, with ``want_sum``, x + residual (bf16 [R, H])."""
    rows, hidden = x.shape
    out = torch.empty_like(x)
    total = torch.empty_like(x) if want_sum else None
    a = _lib.SgAddRmsNormArgs()
    a.num_rows, a.hidden, a.eps = rows, hidden, float(eps)
    a.x_dev, a.x_stride = x.data_ptr(), x.stride(0)
    if residual is not None:
        a.residual_dev, a.residual_stride = residual.data_ptr(), residual.stride(0)
    a.weight_dev = weight.data_ptr()
    a.out_dev, a.out_stride = out.data_ptr(), out.stride(0)
    if total is not None:
        a.residual_out_dev, a.residual_out_stride = total.data_ptr(), total.stride(0)
    _lib.check(_lib.load().sg_add_rmsnorm(ctypes.byref(a), _stream()), "sg_add_rmsnorm")
    return (out, total) if want_sum else out


def qk_norm_rope(qkv: torch.Tensor, num_q_heads: int, num_kv_heads: int, head_dim: int,
                 q_norm: torch.Tensor, k_norm: torch.Tensor, inv_freq: torch.Tensor,
                 positions: torch.Tensor, eps: float):
    """q [R, Hq, D] and k, v [Hkv, R, D] (bf16) from the merged projection."""
    rows = qkv.shape[0]
    q = torch.empty((rows, num_q_heads, head_dim), dtype=qkv.dtype, device=qkv.device)
    kv = torch.empty((2, num_kv_heads, rows, head_dim), dtype=qkv.dtype, device=qkv.device)
    a = _lib.SgQkNormRopeArgs()
    a.num_rows, a.num_q_heads, a.num_kv_heads, a.head_dim = rows, num_q_heads, num_kv_heads, head_dim
    a.eps = float(eps)
    a.qkv_dev, a.qkv_row_stride = qkv.data_ptr(), qkv.stride(0)
    a.q_norm_dev, a.k_norm_dev = q_norm.data_ptr(), k_norm.data_ptr()
    a.inv_freq_dev, a.positions_dev = inv_freq.data_ptr(), positions.data_ptr()
    a.q_out_dev, a.q_row_stride = q.data_ptr(), q.stride(0)
    a.k_out_dev, a.v_out_dev = kv[0].data_ptr(), kv[1].data_ptr()
    a.kv_head_stride = kv.stride(1)
    _lib.check(_lib.load().sg_qk_norm_rope(ctypes.byref(a), _stream()), "sg_qk_norm_rope")
    return q, kv[0], kv[1]


def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    rows, width = gate_up.shape
    out = torch.empty((rows, width // 2), dtype=gate_up.dtype, device=gate_up.device)
    _lib.check(_lib.load().sg_silu_mul(gate_up.data_ptr(), gate_up.stride(0), rows, width // 2,
                                       out.data_ptr(), out.stride(0), _stream()),
               "sg_silu_mul")
    return out


def gather_rows(sources: Sequence[torch.Tensor], index: torch.Tensor) -> torch.Tensor:
    """[K, L*H]: the rows ``index`` of each [R, H] source, side by side."""
    first = sources[0]
    rows, width = first.shape
    for t in sources:
        if t.shape != first.shape or t.stride() != first.stride() or t.dtype != torch.bfloat16:
            raise ValueError("Feature sources must share shape, strides and dtype bf16")
    pointers = ops.pointer_array(list(sources), first.device)
    out = torch.empty((index.numel(), len(sources) * width), dtype=first.dtype,
                      device=first.device)
    status = torch.zeros(1, dtype=torch.int32, device=first.device)
    _lib.check(_lib.load().sg_gather_rows(pointers.data_ptr(), len(sources), first.stride(0),
                                          width, rows, index.data_ptr(), index.numel(),
                                          out.data_ptr(), out.stride(0), status.data_ptr(),
                                          _stream()), "sg_gather_rows")
    out.status = status  # SG_EINVAL when an index was out of range
    return out


@dataclass
class _Layer:
    ln1: torch.Tensor
    wqkv: torch.Tensor   # [(Hq + 2 Hkv) D, H]
    q_norm: torch.Tensor
    k_norm: torch.Tensor
    wo: torch.Tensor     # [H, Hq D]
    ln2: torch.Tensor
    wgu: torch.Tensor    # [2 I, H]
    wd: torch.Tensor     # [H, I]


class _Head:
    """The LM head as the decode loop calls it (``get_output_embeddings()``)."""

    def __init__(self, weight: torch.Tensor):
        self.weight = weight
        self.bias = None

    def __call__(self, hidden: torch.Tensor) -> torch.Tensor:
        return torch.matmul(hidden, self.weight.T)


class _Decoder:
    def __init__(self, stack: "Qwen3TargetStack"):
        self._stack = stack

    def __call__(self, **kwargs):
        return self._stack.forward(**kwargs)


class Qwen3TargetStack:
    """Qwen3 target decoder on the HIP verification kernels (see the module
    docstring)."""

    def __init__(self, *, embed: torch.Tensor, layers: Sequence[_Layer], norm: torch.Tensor,
                 lm_head: torch.Tensor, num_q_heads: int, num_kv_heads: int, head_dim: int,
                 rope_theta: float, eps: float):
        self.embed = embed
        self.layers = list(layers)
        self.norm = norm
        self.lm_head = _Head(lm_head)
        self.num_q_heads, self.num_kv_heads, self.head_dim = num_q_heads, num_kv_heads, head_dim
        self.eps = float(eps)
        # Rotary inverse frequencies as transformers computes them (fp32).
        exponents = torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim
        self.inv_freq = (1.0 / (float(rope_theta) ** exponents)).to(embed.device)
        self.model = _Decoder(self)

    @classmethod
    def from_transformers(cls, model) -> "Qwen3TargetStack":
        cfg = model.config
        if getattr(cfg, "model_type", "qwen3") != "qwen3":
            raise ValueError("Qwen3TargetStack takes a Qwen3 causal LM")
        if getattr(cfg, "rope_scaling", None) not in (None, {}) and \
                (cfg.rope_scaling or {}).get("rope_type", "default") != "default":
            raise ValueError("Only the default rotary embedding is implemented")
        base = model.model
        dtype = torch.bfloat16

        def w(t):
            return t.detach().to(dtype).contiguous()

        layers = []
        for layer in base.layers:
            attn, mlp = layer.self_attn, layer.mlp
            if any(getattr(m, "bias", None) is not None
                   for m in (attn.q_proj, attn.k_proj, attn.v_proj, attn.o_proj)):
                raise ValueError("Projections with bias are not implemented")
            layers.append(_Layer(
                ln1=w(layer.input_layernorm.weight),
                wqkv=w(torch.cat([attn.q_proj.weight, attn.k_proj.weight,
                                  attn.v_proj.weight], 0)),
                q_norm=w(attn.q_norm.weight), k_norm=w(attn.k_norm.weight),
                wo=w(attn.o_proj.weight), ln2=w(layer.post_attention_layernorm.weight),
                wgu=w(torch.cat([mlp.gate_proj.weight, mlp.up_proj.weight], 0)),
                wd=w(mlp.down_proj.weight)))
        theta = getattr(cfg, "rope_theta", None)
        if theta is None:
            theta = (getattr(cfg, "rope_parameters", None) or {}).get("rope_theta", 10000.0)
        return cls(embed=w(base.embed_tokens.weight), layers=layers, norm=w(base.norm.weight),
                   lm_head=w(model.lm_head.weight), num_q_heads=cfg.num_attention_heads,
                   num_kv_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim,
                   rope_theta=theta, eps=cfg.rms_norm_eps)

    # The decode loop reads the device and dtype from the first parameter.
    def parameters(self):
        yield self.embed

    def get_output_embeddings(self):
        return self.lm_head

    def forward(self, *, input_ids: torch.Tensor, position_ids: torch.Tensor, attention_mask,
                past_key_values, use_cache: bool = True, output_hidden_states: bool = False,
                **kwargs):
        mask = attention_mask.get("full_attention") if isinstance(attention_mask, dict) \
            else attention_mask
        if not isinstance(mask, attention.PackedTreeMask):
            raise ValueError("The HIP target stack needs the wave's PackedTreeMask")
        if input_ids.dim() != 2 or input_ids.shape[0] != 1:
            raise ValueError("Packed verification runs one packed sequence")
        cache = past_key_values
        rows = input_ids.shape[1]
        if rows != mask.num_rows:
            raise ValueError("Packed rows disagree with the tree mask")
        positions = position_ids.reshape(-1).to(torch.int64).contiguous()
        hq, hkv, d = self.num_q_heads, self.num_kv_heads, self.head_dim
        plan = mask.plan(hq, hkv, d)
        x = torch.nn.functional.embedding(input_ids[0], self.embed)
        states = [x] if output_hidden_states else None
        residual = None
        carry = x   # what the next add+RMSNorm adds to the residual stream
        for index, layer in enumerate(self.layers):
            h, residual = add_rmsnorm(carry, layer.ln1, self.eps, residual, want_sum=True)
            if states is not None and index > 0:
                states.append(residual)
            qkv = torch.matmul(h, layer.wqkv.T)
            q, k, v = qk_norm_rope(qkv, hq, hkv, d, layer.q_norm, layer.k_norm, self.inv_freq,
                                   positions, self.eps)
            k_new, v_new = cache.update(k[None], v[None], index)
            attn = torch.empty((rows, hq, d), dtype=x.dtype, device=x.device)
            ops.tree_attention(q, mask.pool.key_storage[index], mask.pool.value_storage[index],
                               k_new[0].transpose(0, 1), v_new[0].transpose(0, 1),
                               mask.row_offset, mask.prefix_start, mask.prefix_len, mask.parent,
                               plan, out=attn, scale=d ** -0.5)
            o = torch.matmul(attn.view(rows, hq * d), layer.wo.T)
            h, residual = add_rmsnorm(o, layer.ln2, self.eps, residual, want_sum=True)
            carry = torch.matmul(silu_mul(torch.matmul(h, layer.wgu.T)), layer.wd.T)
        final = add_rmsnorm(carry, self.norm, self.eps, residual)
        if states is not None:
            states.append(final)
        return SimpleNamespace(
            last_hidden_state=final[None],
            hidden_states=tuple(t[None] for t in states) if states is not None else None,
            past_key_values=cache if use_cache else None)

    def features(self, output, target_layer_ids: Sequence[int],
                 keep_index: torch.Tensor) -> torch.Tensor:
        """Draft features of the kept rows: ``hidden_states[i + 1]`` rows
        ``keep_index`` of every target layer i, concatenated along the feature
        dimension (continuous_tree_block_decode.py:2149-2158), [1, K, L*H]."""
        if output.hidden_states is None:
            raise ValueError("Run the stack with output_hidden_states=True")
        sources = [output.hidden_states[i + 1][0] for i in target_layer_ids]
        gathered = gather_rows(sources, keep_index.to(torch.int32).contiguous())
        return gathered[None]
