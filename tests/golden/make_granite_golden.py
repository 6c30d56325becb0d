"""Writes tests/golden/granite_tiny.npz: logits and router logits of the transformers GraniteMoeForCausalLM
(transformers 5.15.0, float32, teacher forcing over 70 tokens) loaded with the seeded synthetic f32 weights that
moert.SynthModel builds. The reference validated its CPU path against this same model class
(tools/ref_logits.py, tools/ref_moe_block.py in the reference); here it pins the model composition of the oracle:
embedding multiplier, residual placement, rotate_half RoPE, GQA head mapping, top-k-then-softmax routing and the
tied head divided by logits_scaling.

Shapes follow the reference's synthetic test model (rust/moe-rt/tests/common/mod.rs:79-131): hidden 256, inter 128,
2 layers, 4 query / 2 KV heads of 64, 4 experts top-2, odd vocabulary 33, multipliers 2.0 / 0.5 / 0.125 / 4.0.

Run from the repository root after building libmoert.so:  python tests/golden/make_granite_golden.py
"""
import os
import sys

import numpy as np
import torch
import transformers

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "lastro-rust_amd"))
import moert  # noqa: E402

SEED = 77
STD = 0.1
T = 70
CFG = dict(hidden=256, inter=128, layers=2, heads=4, kv_heads=2, head_dim=64, vocab=33, experts=4, top_k=2,
           rope_theta=10000.0, eps=1e-6, embedding_multiplier=2.0, residual_multiplier=0.5,
           attention_multiplier=0.125, logits_scaling=4.0)


def main():
    cfg = moert.Config(**CFG)
    m = moert.SynthModel(cfg, seed=SEED, wdtype=moert.F32, embed_dtype=moert.F32, std=STD)
    a = m.arrays
    hf_cfg = transformers.GraniteMoeConfig(
        vocab_size=cfg.vocab, hidden_size=cfg.hidden, intermediate_size=cfg.inter, num_hidden_layers=cfg.layers,
        num_attention_heads=cfg.heads, num_key_value_heads=cfg.kv_heads, num_local_experts=cfg.experts,
        num_experts_per_tok=cfg.top_k, max_position_embeddings=256, rms_norm_eps=cfg.eps,
        rope_parameters={"rope_theta": cfg.rope_theta, "rope_type": "default"}, tie_word_embeddings=True,
        embedding_multiplier=cfg.embedding_multiplier, residual_multiplier=cfg.residual_multiplier,
        attention_multiplier=cfg.attention_multiplier, logits_scaling=cfg.logits_scaling, attention_bias=False,
        pad_token_id=0, bos_token_id=0, eos_token_id=0)
    model = transformers.GraniteMoeForCausalLM(hf_cfg).eval().to(torch.float32)
    H, I, E, d = cfg.hidden, cfg.inter, cfg.experts, cfg.head_dim
    qd, kvd = cfg.heads * d, cfg.kv_heads * d
    sd = {"model.embed_tokens.weight": a["embed"].reshape(cfg.vocab, H), "model.norm.weight": a["norm"]}
    for l in range(cfg.layers):
        p = f"model.layers.{l}"
        sd[f"{p}.input_layernorm.weight"] = a[f"{l}.ln_attn"]
        sd[f"{p}.post_attention_layernorm.weight"] = a[f"{l}.ln_moe"]
        sd[f"{p}.self_attn.q_proj.weight"] = a[f"{l}.q"].reshape(qd, H)
        sd[f"{p}.self_attn.k_proj.weight"] = a[f"{l}.k"].reshape(kvd, H)
        sd[f"{p}.self_attn.v_proj.weight"] = a[f"{l}.v"].reshape(kvd, H)
        sd[f"{p}.self_attn.o_proj.weight"] = a[f"{l}.o"].reshape(H, qd)
        sd[f"{p}.block_sparse_moe.router.weight"] = a[f"{l}.router"].reshape(E, H)
        sd[f"{p}.block_sparse_moe.experts.gate_up_proj"] = a[f"{l}.gate_up"].reshape(E, 2 * I, H)
        sd[f"{p}.block_sparse_moe.experts.down_proj"] = a[f"{l}.down"].reshape(E, H, I)
    sd = {k: torch.from_numpy(np.array(v, np.float32)) for k, v in sd.items()}
    sd["lm_head.weight"] = sd["model.embed_tokens.weight"]
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected, unexpected
    assert all(k == "lm_head.weight" for k in missing), missing
    rng = np.random.default_rng(SEED)
    tokens = rng.integers(0, cfg.vocab, T).astype(np.int32)
    ids = torch.from_numpy(tokens.astype(np.int64))[None]

    def run():
        captured = []
        hooks = [layer.block_sparse_moe.router.register_forward_hook(lambda _m, _i, o: captured.append(o[2]))
                 for layer in model.model.layers]
        with torch.inference_mode():
            out = model(ids, use_cache=False)
        for h in hooks:
            h.remove()
        return out.logits[0].float().numpy(), np.stack([r.float().numpy().reshape(T, E) for r in captured])

    model.config._attn_implementation = "eager"
    logits, router = run()
    # Same model with K (after RoPE) and V rounded to fp16, as the engine's KV cache stores them.
    from transformers.models.granitemoe import modeling_granitemoe as mg

    eager = mg.eager_attention_forward

    def fp16_kv_attention(module, q, k, v, mask, *args, **kw):
        return eager(module, q, k.half().float(), v.half().float(), mask, *args, **kw)

    mg.eager_attention_forward = fp16_kv_attention  # the eager path looks the function up at call time
    try:
        logits16, router16 = run()
    finally:
        mg.eager_attention_forward = eager
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "granite_tiny.npz")
    np.savez(path, tokens=tokens, logits=logits.astype(np.float32), router_logits=router.astype(np.float32),
             logits_fp16kv=logits16.astype(np.float32), router_logits_fp16kv=router16.astype(np.float32),
             seed=np.int64(SEED), std=np.float32(STD))
    print(f"wrote {path}: logits {logits.shape}, router {router.shape}, transformers {transformers.__version__}")


if __name__ == "__main__":
    main()
