"""Whole-model logits of the serving model on the HIP path against the oracle.

The reference pins its batch decode at the model level: logits of every
decode step, compared with single-request decode and with a dense
recomputation (tests/model/test_qwen2_batch_decode.py:100-170). Here the
24-layer Qwen2.5-0.5B-architecture model of the serving workload
(workloads.qwen05b_serving: random init from its seed) runs four of that
workload's requests through the runtime (Scheduler -> build_model_batch ->
execute_model_batch: one packed varlen prefill, then five batched decode
steps with the fused rotary decode kernel) under teacher forcing: after each
step every request is fed a fixed random token rather than its argmax, so the
GPU run and the oracle see identical inputs whatever either would pick. Every
request's logits row of every step (prefill's last position, then each
decode) is compared with oracle.qwen2_model.OracleQwen2.teacher_forced_logits
on the CPU (the reference's model restated, dense causal prompt pass and
contiguous K/V, no paging):

- FP32: max-abs error at most FP32_TOL over all 151,936 logits of all 24 rows,
  and the argmax equal wherever the oracle's top-2 margin exceeds
  FP32_MARGIN;
- BF16 (FP32 RMSNorm statistics and softmax): max-abs error at most
  BF16_TOL, and the argmax equal wherever the oracle's top-2 margin exceeds
  BF16_MARGIN. The two sides round their bf16 GEMMs in different orders, and
  the differences compound over 24 layers; the logits reach about 3.2 here.
- FP16 (the same, in fp16: the matrix-core prefill and one-launch decode
  with fp16 operands): max-abs error at most FP16_TOL, the argmax equal
  wherever the margin exceeds FP16_MARGIN.
"""

from __future__ import annotations

import copy

import pytest
import torch

from mini_llm_runtime_amd import workloads
from mini_llm_runtime_amd.model.qwen2 import TinyQwen2Config, TinyQwen2ForCausalLM
from mini_llm_runtime_amd.runtime.model_runner import build_model_batch, execute_model_batch
from mini_llm_runtime_amd.runtime.paged_kv_cache import PagedKVCache
from mini_llm_runtime_amd.runtime.request import Request
from mini_llm_runtime_amd.runtime.scheduler import Scheduler
from oracle.qwen2_model import OracleQwen2

pytestmark = pytest.mark.gpu

# FP32: the reference's own model-level bar (1e-5); argmax checked wherever
# the margin is ten times that. BF16: four bf16 ulps of logits in [2, 4)
# (measured: at most 3.5e-2, about two ulps); argmax checked wherever the
# margin is twice the tolerance.
FP32_TOL, FP32_MARGIN, FP32_MIN_CHECKS = 1e-5, 1e-4, 20
BF16_TOL, BF16_MARGIN, BF16_MIN_CHECKS = 6.25e-2, 0.125, 8
# FP16: four fp16 ulps of logits in [2, 4) (measured: at most 3.9e-3, about
# two ulps); argmax checked wherever the margin is twice the tolerance.
FP16_TOL, FP16_MARGIN, FP16_MIN_CHECKS = 7.8125e-3, 1.5625e-2, 12
DECODE_STEPS = 5
REQUESTS = ("init0", "init7", "init2", "arr0")  # prompts of 218, 687, 942, 1024 tokens


@pytest.fixture(scope="module")
def serving_model():
    w = workloads.qwen05b_serving()
    cfg = TinyQwen2Config(**w.config)
    torch.manual_seed(w.model_seed)
    model = TinyQwen2ForCausalLM(cfg).float().eval()
    prompts = {f"init{i}": p for i, (p, _) in enumerate(w.initial)}
    prompts.update({f"arr{i}": p for i, (p, _) in enumerate(w.arrivals)})
    return cfg, model, {rid: prompts[rid] for rid in REQUESTS}


def run_teacher_forced(model, cfg, prompts, forced, dtype, device):
    """Logits rows [1 + DECODE_STEPS, vocab] per request from the runtime."""
    need = sum(-(-(len(p) + DECODE_STEPS + 1) // 16) for p in prompts.values())
    cache = PagedKVCache(cfg.num_hidden_layers, need + 16, 16, cfg.num_key_value_heads,
                         cfg.head_dim, dtype=dtype, device=device)
    scheduler = Scheduler(max_num_batched_tokens=4096, max_num_seqs=len(prompts),
                          kv_cache=cache)
    for rid, prompt in prompts.items():
        scheduler.add_request(Request(rid, prompt, DECODE_STEPS + 1, 0.0))
    rows = {rid: [] for rid in prompts}
    with torch.no_grad():
        for step in range(DECODE_STEPS + 1):
            out = scheduler.schedule()
            batch = build_model_batch(out, block_size=16, device=device)
            logits = execute_model_batch(model, batch, cache)
            qsl = batch.query_start_loc.tolist()
            assert sorted(batch.request_ids) == sorted(prompts), step
            for i, rid in enumerate(batch.request_ids):
                rows[rid].append(logits[qsl[i + 1] - 1].double().cpu())
            scheduler.update_after_model(
                out, {rid: forced[rid][step] for rid in batch.request_ids}, set())
    assert not scheduler.running and not scheduler.waiting
    return {rid: torch.stack(r) for rid, r in rows.items()}


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16],
                         ids=["fp32", "bf16", "fp16"])
def test_qwen05b_24_layer_teacher_forced_logits(device, serving_model, dtype):
    cfg, model, prompts = serving_model
    gen = torch.Generator().manual_seed(17)
    forced = {rid: torch.randint(0, cfg.vocab_size, (DECODE_STEPS + 1,), generator=gen).tolist()
              for rid in prompts}
    oracle = OracleQwen2(model.state_dict(), cfg, dtype=dtype)
    gpu_model = copy.deepcopy(model).to(device=device, dtype=dtype).eval()
    got = run_teacher_forced(gpu_model, cfg, prompts, forced, dtype, device)
    tol, margin_bar, min_checks = {
        torch.float32: (FP32_TOL, FP32_MARGIN, FP32_MIN_CHECKS),
        torch.bfloat16: (BF16_TOL, BF16_MARGIN, BF16_MIN_CHECKS),
        torch.float16: (FP16_TOL, FP16_MARGIN, FP16_MIN_CHECKS)}[dtype]
    worst, scale, checked = 0.0, 0.0, 0
    with torch.no_grad():
        for rid, prompt in prompts.items():
            want = oracle.teacher_forced_logits(prompt, forced[rid][:DECODE_STEPS]).double()
            err = (got[rid] - want).abs().max(dim=-1).values
            worst = max(worst, err.max().item())
            scale = max(scale, want.abs().max().item())
            top = want.topk(2, dim=-1)
            for step in range(DECODE_STEPS + 1):
                margin = (top.values[step, 0] - top.values[step, 1]).item()
                print(f"{str(dtype)[6:]} {rid} step {step}: max-abs {err[step].item():.3e}, "
                      f"oracle margin {margin:.3e}")
                if margin > margin_bar:
                    assert int(got[rid][step].argmax()) == int(top.indices[step, 0]), (rid, step)
                    checked += 1
    print(f"{str(dtype)[6:]}: worst max-abs {worst:.3e} over logits up to {scale:.2f}; "
          f"{checked} argmax checks")
    assert worst <= tol
    assert checked >= min_checks
