"""CPU restatement of the reference's Qwen2 causal LM (oracle; tests only).

Follows src/mini_llm_runtime/model/qwen2.py:
- Qwen2RMSNorm (:88-123): x * rsqrt(mean(x^2) + eps), statistics in FP32 for
  FP16/BF16 inputs, product weight * normalized taken in the input dtype;
- Qwen2MLP (:768-792): down(silu(gate(x)) * up(x)), no biases;
- Qwen2DecoderLayer.forward (:815-833): pre-norm attention and MLP, residuals;
- TinyQwen2Model.forward (:943-1003): embedding, layers, final norm, with the
  reference's dense causal attention (:282-370);
- TinyQwen2ForCausalLM (:1170-1240): lm_head (tied to the embedding when the
  config says so).

``dense_greedy`` is the reference integration tests' expected-token helper
(tests/integration/test_qwen2_5_continuous_batching.py:61-76): recompute the
whole sequence every step, take the argmax of the last row.
``cached_greedy`` gives the same tokens with per-layer contiguous K/V (one new
row per step), cheap enough for long prompts; the two agree on small inputs
(tests/oracle_pins.py). Both are independent of paging and batching: a
continuous-batching run must reproduce each request's tokens.

Weights: the model's state_dict (reference names), as CPU tensors.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import qwen2_attention as qa


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    dtype = x.dtype
    stats = torch.float32 if dtype in (torch.float16, torch.bfloat16) else dtype
    h = x.to(stats)
    normalized = h * torch.rsqrt(h.square().mean(dim=-1, keepdim=True) + eps)
    return weight.to(dtype) * normalized.to(dtype)


def mlp(x: torch.Tensor, gate_w, up_w, down_w) -> torch.Tensor:
    return F.linear(F.silu(F.linear(x, gate_w)) * F.linear(x, up_w), down_w)


class OracleQwen2:
    def __init__(self, state_dict: dict, config, dtype: torch.dtype | None = None):
        sd = {k: v.detach().to("cpu") for k, v in state_dict.items()}
        if dtype is not None:
            sd = {k: v.to(dtype) for k, v in sd.items()}
        self.cfg = config
        self.dims = (config.num_attention_heads, config.num_key_value_heads,
                     config.head_dim, config.rope_theta)
        # A reference model cast with .to(dtype) holds its rotary inv_freq
        # buffers in that dtype (qwen2_attention.rope_tables).
        self.freq_dtype = dtype
        self.embed = sd["model.embed_tokens.weight"]
        self.norm_w = sd["model.norm.weight"]
        self.lm_head = sd.get("lm_head.weight", self.embed)
        self.layers = []
        for i in range(config.num_hidden_layers):
            p = f"model.layers.{i}."
            a = p + "self_attn."
            self.layers.append({
                "in_norm": sd[p + "input_layernorm.weight"],
                "post_norm": sd[p + "post_attention_layernorm.weight"],
                "attn": {"q_w": sd[a + "qkv_proj.q_proj.weight"],
                         "q_b": sd[a + "qkv_proj.q_proj.bias"],
                         "k_w": sd[a + "qkv_proj.k_proj.weight"],
                         "k_b": sd[a + "qkv_proj.k_proj.bias"],
                         "v_w": sd[a + "qkv_proj.v_proj.weight"],
                         "v_b": sd[a + "qkv_proj.v_proj.bias"],
                         "o_w": sd[a + "o_proj.weight"]},
                "gate": sd[p + "mlp.gate_proj.weight"],
                "up": sd[p + "mlp.up_proj.weight"],
                "down": sd[p + "mlp.down_proj.weight"],
            })

    def _mlp_block(self, h, layer):
        return h + mlp(rms_norm(h, layer["post_norm"], self.cfg.rms_norm_eps),
                       layer["gate"], layer["up"], layer["down"])

    def _logits(self, h):
        return F.linear(rms_norm(h, self.norm_w, self.cfg.rms_norm_eps), self.lm_head)

    def forward(self, tokens: list[int]) -> torch.Tensor:
        """Logits [S, vocab] of the whole sequence (dense causal attention)."""
        hq, hkv, d, theta = self.dims
        ids = torch.tensor([tokens], dtype=torch.long)
        pos = torch.arange(len(tokens), dtype=torch.long).unsqueeze(0)
        h = F.embedding(ids, self.embed)
        for layer in self.layers:
            x = rms_norm(h, layer["in_norm"], self.cfg.rms_norm_eps)
            q, k, v = qa.qkv_rope(x, pos, layer["attn"], hq, hkv, d, theta, self.freq_dtype)
            h = h + F.linear(qa.dense_causal(q, k, v, d ** -0.5), layer["attn"]["o_w"])
            h = self._mlp_block(h, layer)
        return self._logits(h)[0]

    def dense_greedy(self, prompt: list[int], max_new_tokens: int) -> list[int]:
        tokens, out = list(prompt), []
        for _ in range(max_new_tokens):
            nxt = int(self.forward(tokens)[-1].argmax())
            out.append(nxt)
            tokens.append(nxt)
        return out

    def _prompt_pass(self, prompt: list[int]):
        """The prompt in one dense causal pass: the logits row of its last
        position, and per layer the contiguous K/V rows [T, Hkv, D]."""
        hq, hkv, d, theta = self.dims
        ks: list[torch.Tensor] = []
        vs: list[torch.Tensor] = []
        ids = torch.tensor([prompt], dtype=torch.long)
        pos = torch.arange(len(prompt), dtype=torch.long).unsqueeze(0)
        h = F.embedding(ids, self.embed)
        for layer in self.layers:
            x = rms_norm(h, layer["in_norm"], self.cfg.rms_norm_eps)
            q, k, v = qa.qkv_rope(x, pos, layer["attn"], hq, hkv, d, theta, self.freq_dtype)
            ks.append(k[0])
            vs.append(v[0])
            h = h + F.linear(qa.dense_causal(q, k, v, d ** -0.5), layer["attn"]["o_w"])
            h = self._mlp_block(h, layer)
        return self._logits(h)[0, -1], ks, vs

    def _decode_row(self, token: int, p: int, ks: list, vs: list) -> torch.Tensor:
        """One decode step: `token` at position `p` attends over every K/V row
        so far plus its own (appended to ks/vs); its logits row."""
        hq, hkv, d, theta = self.dims
        group, scale = hq // hkv, d ** -0.5
        h = F.embedding(torch.tensor([[token]]), self.embed)
        posn = torch.tensor([[p]], dtype=torch.long)
        for i, layer in enumerate(self.layers):
            x = rms_norm(h, layer["in_norm"], self.cfg.rms_norm_eps)
            q, k, v = qa.qkv_rope(x, posn, layer["attn"], hq, hkv, d, theta, self.freq_dtype)
            ks[i] = torch.cat([ks[i], k[0]])
            vs[i] = torch.cat([vs[i], v[0]])
            kk = ks[i].repeat_interleave(group, dim=-2).transpose(0, 1)   # [Hq, T, D]
            vv = vs[i].repeat_interleave(group, dim=-2).transpose(0, 1)
            scores = (q[0, 0].unsqueeze(1) @ kk.transpose(-2, -1)) * scale  # [Hq, 1, T]
            sm = torch.float32 if scores.dtype in (torch.float16, torch.bfloat16) \
                else scores.dtype
            probs = torch.softmax(scores, dim=-1, dtype=sm).to(vv.dtype)
            att = (probs @ vv).reshape(1, 1, hq * d)
            h = h + F.linear(att, layer["attn"]["o_w"])
            h = self._mlp_block(h, layer)
        return self._logits(h)[0, -1]

    def cached_greedy(self, prompt: list[int], max_new_tokens: int,
                      margins: list | None = None) -> list[int]:
        """Greedy tokens with contiguous per-layer K/V: the prompt in one dense
        causal pass, then one row per step attending over all rows so far.
        ``margins``, when given, receives (top1 - top2 logit, second-best
        token) per step: a run in another precision or reduction order may
        only pick differently where that margin is within its rounding."""
        def pick(logits_row: torch.Tensor) -> int:
            top = logits_row.topk(2)
            if margins is not None:
                margins.append((float(top.values[0] - top.values[1]), int(top.indices[1])))
            return int(top.indices[0])

        row, ks, vs = self._prompt_pass(prompt)
        out = [pick(row)]
        while len(out) < max_new_tokens:
            out.append(pick(self._decode_row(out[-1], len(prompt) + len(out) - 1, ks, vs)))
        return out

    def teacher_forced_logits(self, prompt: list[int], forced: list[int]) -> torch.Tensor:
        """Logits rows [1 + len(forced), vocab]: the prompt's last position,
        then the row of each forced token fed in turn at the next position
        (whatever the model would have picked), as the reference's batch
        decode test drives its model (tests/model/test_qwen2_batch_decode.py:
        100-170)."""
        row, ks, vs = self._prompt_pass(prompt)
        rows = [row]
        for i, token in enumerate(forced):
            rows.append(self._decode_row(token, len(prompt) + i, ks, vs))
        return torch.stack(rows)
