"""Plant plausible mistakes in copies of the oracle; the pins must catch each.

A mutant is oracle/paged_attention.py with one source edit, executed as a
fresh module on the CPU. If no pin check fails for a mutant, the pins would
not notice that mistake in the oracle either, and this test fails.
"""

from __future__ import annotations

import inspect
import types

import pytest

import oracle.paged_attention as pa

import oracle_pins

MUTATIONS = {
    # GQA: query head h reads KV head h % Hkv instead of h // group.
    "gqa-map-tiled-not-interleaved": (
        "k = k_cache[physical, offsets].transpose(1, 2).repeat_interleave(group, dim=1)\n"
        "    v = v_cache[physical, offsets].transpose(1, 2).repeat_interleave(group, dim=1)",
        "k = k_cache[physical, offsets].transpose(1, 2).repeat(1, group, 1, 1)\n"
        "    v = v_cache[physical, offsets].transpose(1, 2).repeat(1, group, 1, 1)",
    ),
    "dropped-decode-scale": (
        "scores = torch.matmul(q.unsqueeze(2), k.transpose(-2, -1)) * scale",
        "scores = torch.matmul(q.unsqueeze(2), k.transpose(-2, -1))",
    ),
    "length-mask-off-by-one": (
        "live = pos.unsqueeze(0) < seq_lens.unsqueeze(1)",
        "live = pos.unsqueeze(0) < seq_lens.unsqueeze(1) - 1",
    ),
    "block-offset-swapped": (
        "keys.append(k_cache[block][pos % block_size])",
        "keys.append(k_cache[block][(pos + 1) % block_size])",
    ),
    "causal-mask-strict": (
        "visible = positions.unsqueeze(0) <= query_pos.unsqueeze(1)\n"
        "        scores = scores.to(torch.float32)",
        "visible = positions.unsqueeze(0) < query_pos.unsqueeze(1)\n"
        "        scores = scores.to(torch.float32)",
    ),
    "online-rescale-dropped": (
        "acc = acc * rescale + weights @ values.to(torch.float32)",
        "acc = acc + weights @ values.to(torch.float32)",
    ),
    "prefill-prefix-ignored": (
        "query_pos = prefix_len + torch.arange(chunk, device=q.device)",
        "query_pos = torch.arange(chunk, device=q.device)",
    ),
    "dense-slot-uses-offset-only": (
        "return table[positions // block_size] * block_size + positions % block_size",
        "return table[positions // block_size] * block_size",
    ),
}


def make_mutant(name: str) -> types.ModuleType:
    before, after = MUTATIONS[name]
    source = inspect.getsource(pa)
    assert source.count(before) == 1, f"mutation site for {name} not found exactly once"
    module = types.ModuleType(f"oracle_mutant_{name}")
    exec(compile(source.replace(before, after), module.__name__, "exec"), module.__dict__)
    return module


@pytest.mark.parametrize("name", sorted(MUTATIONS))
def test_pins_catch_planted_mistake(name):
    mutant = make_mutant(name)
    caught = []
    for check in oracle_pins.ALL_CHECKS:
        try:
            check(mutant)
        except (AssertionError, IndexError, RuntimeError, ValueError):
            caught.append(check.__name__)
    assert caught, f"no pin detects the planted mistake {name!r}"


# The same for the Qwen2 attention callers (oracle/qwen2_attention.py).
QWEN2_MUTATIONS = {
    "rope-sign-flipped": (
        "turned = torch.cat((-x[..., half:], x[..., :half]), dim=-1)",
        "turned = torch.cat((x[..., half:], -x[..., :half]), dim=-1)",
    ),
    "rope-adjacent-pairs": (
        "turned = torch.cat((-x[..., half:], x[..., :half]), dim=-1)",
        "turned = torch.stack((-x[..., 1::2], x[..., ::2]), dim=-1).flatten(-2)",
    ),
    "rope-angles-not-duplicated": (
        "angles = torch.cat((angles, angles), dim=-1)",
        "angles = torch.cat((angles, angles.flip(-1)), dim=-1)",
    ),
    "k-bias-dropped": (
        'k = torch.nn.functional.linear(hidden, w["k_w"], w["k_b"])',
        'k = torch.nn.functional.linear(hidden, w["k_w"])',
    ),
}


@pytest.mark.parametrize("name", sorted(QWEN2_MUTATIONS))
def test_qwen2_pins_catch_planted_mistake(name):
    import oracle.qwen2_attention as qa
    before, after = QWEN2_MUTATIONS[name]
    source = inspect.getsource(qa)
    assert source.count(before) == 1, f"mutation site for {name} not found exactly once"
    module = types.ModuleType(f"oracle.qwen2_mutant_{name.replace('-', '_')}")
    module.__package__ = "oracle"
    exec(compile(source.replace(before, after), module.__name__, "exec"), module.__dict__)
    caught = []
    for check in oracle_pins.QWEN2_CHECKS:
        try:
            check(module)
        except (AssertionError, IndexError, RuntimeError, ValueError):
            caught.append(check.__name__)
    assert caught, f"no pin detects the planted mistake {name!r}"


# And for the whole model (oracle/qwen2_model.py).
MODEL_MUTATIONS = {
    "rmsnorm-eps-dropped": (
        "normalized = h * torch.rsqrt(h.square().mean(dim=-1, keepdim=True) + eps)",
        "normalized = h * torch.rsqrt(h.square().mean(dim=-1, keepdim=True))",
    ),
    "mlp-gate-up-swapped": (
        "return F.linear(F.silu(F.linear(x, gate_w)) * F.linear(x, up_w), down_w)",
        "return F.linear(F.silu(F.linear(x, up_w)) * F.linear(x, gate_w), down_w)",
    ),
    "final-norm-skipped": (
        "return F.linear(rms_norm(h, self.norm_w, self.cfg.rms_norm_eps), self.lm_head)",
        "return F.linear(h, self.lm_head)",
    ),
    "decode-row-position-off-by-one": (
        "posn = torch.tensor([[p]], dtype=torch.long)",
        "posn = torch.tensor([[p + 1]], dtype=torch.long)",
    ),
    "teacher-forced-row-skipped": (
        "rows.append(self._decode_row(token, len(prompt) + i, ks, vs))",
        "rows.append(self._decode_row(token, len(prompt) + i + 1, ks, vs))",
    ),
}


@pytest.mark.parametrize("name", sorted(MODEL_MUTATIONS))
def test_model_pins_catch_planted_mistake(name):
    import oracle.qwen2_model as qm
    before, after = MODEL_MUTATIONS[name]
    source = inspect.getsource(qm)
    assert source.count(before) == 1, f"mutation site for {name} not found exactly once"
    module = types.ModuleType(f"oracle.model_mutant_{name.replace('-', '_')}")
    module.__package__ = "oracle"
    exec(compile(source.replace(before, after), module.__name__, "exec"), module.__dict__)
    caught = []
    for check in oracle_pins.MODEL_CHECKS:
        try:
            check(module)
        except (AssertionError, IndexError, RuntimeError, ValueError):
            caught.append(check.__name__)
    assert caught, f"no pin detects the planted mistake {name!r}"
