"""CPU pinning of the oracle's Qwen2 decode-step pieces against transformers.

The reference's model-level decode (``src/triton_kernels/paged_kv.py:690-820``)
runs a transformers Qwen2 model with bnb NF4 base weights and LoRA.  The
installed transformers implementation is an independent statement of the same
network, so the oracle's RMSNorm, RoPE and whole decode step are checked
against it: RMSNorm and RoPE at bf16 (bit-level), the step against a float32
transformers model whose linear weights are the dequantized NF4 values with
the LoRA update folded in (W + s * B @ A), within the bf16 tolerance that the
oracle's intermediate rounding allows.
"""

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits
from oracle.decode import Qwen2DecodeOracle, apply_rope, rmsnorm, rope_tables
from oracle.nf4 import dequantize_nf4, quantize_nf4

from conftest import rel_err

transformers = pytest.importorskip("transformers")
from transformers import Qwen2Config  # noqa: E402
from transformers.models.qwen2.modeling_qwen2 import (  # noqa: E402
    Qwen2ForCausalLM,
    Qwen2RMSNorm,
    Qwen2RotaryEmbedding,
    apply_rotary_pos_emb,
)


def bf16_tensor(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16).copy()).view(torch.bfloat16)


def to_bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def test_rmsnorm_matches_transformers():
    g = np.random.default_rng(0)
    x = f32_to_bf16_bits(g.standard_normal((8, 1536)) * 3.0)
    w = f32_to_bf16_bits(1.0 + 0.1 * g.standard_normal(1536))
    m = Qwen2RMSNorm(1536, eps=1e-6).to(torch.bfloat16)
    with torch.no_grad():
        m.weight.copy_(bf16_tensor(w))
        ref = to_bits(m(bf16_tensor(x)))
    got = rmsnorm(x, w, 1e-6)
    diff = np.abs(got.astype(np.int32) - ref.astype(np.int32))
    assert diff.max() <= 1 and np.mean(diff == 0) >= 0.99


def test_rope_matches_transformers():
    cfg = Qwen2Config(hidden_size=1536, num_attention_heads=12, num_key_value_heads=2,
                      rope_theta=1_000_000.0, max_position_embeddings=4096)
    rot = Qwen2RotaryEmbedding(cfg)
    pos = np.array([0, 1, 7, 511, 1023, 3000])
    g = np.random.default_rng(1)
    q = f32_to_bf16_bits(g.standard_normal((len(pos), 12, 128)))
    k = f32_to_bf16_bits(g.standard_normal((len(pos), 2, 128)))
    xq = bf16_tensor(q)
    cos_t, sin_t = rot(xq, torch.from_numpy(pos)[None, :])
    cos, sin = rope_tables(pos, 128, 1_000_000.0)
    # Tables: the oracle rounds float64 cos/sin once; torch evaluates pow/cos in
    # float32, so an entry may sit one bf16 ulp away at a rounding boundary.
    for t, o in ((cos_t[0], cos), (sin_t[0], sin)):
        d = np.abs(to_bits(t).astype(np.int32) - o.astype(np.int32))
        assert d.max() <= 1 and np.mean(d == 0) >= 0.99
    # Rotation arithmetic: bit-exact on the same tables.
    cb, sb = to_bits(cos_t[0]), to_bits(sin_t[0])
    rq, rk = apply_rotary_pos_emb(xq.transpose(0, 1)[None], bf16_tensor(k).transpose(0, 1)[None],
                                  cos_t, sin_t)
    assert np.array_equal(to_bits(rq[0].transpose(0, 1)), apply_rope(q, cb, sb))
    assert np.array_equal(to_bits(rk[0].transpose(0, 1)), apply_rope(k, cb, sb))


def _tiny_model(seed):
    """Oracle weights of a 2-layer Qwen2-shaped NF4+LoRA model and the matching
    float32 transformers model (dequantized weights, LoRA folded in)."""
    V, H, Hq, Hkv, D, I, L, r, s = 96, 128, 4, 2, 32, 256, 2, 8, 2.0
    g = np.random.default_rng(seed)
    bfb = lambda shape, sd: f32_to_bf16_bits(g.standard_normal(shape) * sd)
    cfg = Qwen2Config(vocab_size=V, hidden_size=H, intermediate_size=I, num_hidden_layers=L,
                      num_attention_heads=Hq, num_key_value_heads=Hkv, head_dim=D,
                      rms_norm_eps=1e-6, rope_theta=10000.0, tie_word_embeddings=False,
                      max_position_embeddings=256, attn_implementation="eager")
    hf = Qwen2ForCausalLM(cfg).float().eval()
    w = dict(embed=bfb((V, H), 1.0), norm=f32_to_bf16_bits(1 + 0.1 * g.standard_normal(H)),
             lm_head=bfb((V, H), 0.05), layers=[])
    sd = {"model.embed_tokens.weight": w["embed"], "model.norm.weight": w["norm"],
          "lm_head.weight": w["lm_head"]}
    dims = dict(q=(Hq * D, H), k=(Hkv * D, H), v=(Hkv * D, H), o=(H, Hq * D), gate=(I, H),
                up=(I, H), down=(H, I))
    for li in range(L):
        e = dict(input_norm=f32_to_bf16_bits(1 + 0.1 * g.standard_normal(H)),
                 post_norm=f32_to_bf16_bits(1 + 0.1 * g.standard_normal(H)))
        pre = f"model.layers.{li}."
        sd[pre + "input_layernorm.weight"] = e["input_norm"]
        sd[pre + "post_attention_layernorm.weight"] = e["post_norm"]
        for name, (n, k) in dims.items():
            packed, absmax = quantize_nf4((g.standard_normal((n, k)) * 0.05).astype(np.float32), 64)
            p = dict(packed=packed, absmax=absmax, n=n, k=k)
            wd = bf16_bits_to_f32(dequantize_nf4(packed, absmax, n * k, 64)).reshape(n, k)
            wd = wd.astype(np.float64)
            if name in ("q", "k", "v", "o"):
                p["A"], p["B"] = bfb((r, k), 0.05), bfb((n, r), 0.05)
                wd = wd + s * bf16_bits_to_f32(p["B"]).astype(np.float64) @ \
                    bf16_bits_to_f32(p["A"]).astype(np.float64)
            if name in ("q", "k", "v"):
                p["bias"] = bfb(n, 0.05)
                sd[pre + f"self_attn.{name}_proj.bias"] = p["bias"]
            mod = "self_attn" if name in ("q", "k", "v", "o") else "mlp"
            sd[pre + f"{mod}.{name}_proj.weight"] = wd.astype(np.float32)
            e[name] = p
        w["layers"].append(e)
    state = {k: torch.from_numpy(bf16_bits_to_f32(v) if v.dtype == np.uint16 else v)
             for k, v in sd.items()}
    hf.load_state_dict(state, strict=True)
    c = dict(hidden=H, n_heads=Hq, n_kv=Hkv, head_dim=D, eps=1e-6, theta=10000.0, blocksize=64,
             scaling=s)
    return w, c, hf


TOL = 1.5e-2  # observed max 0.0076 (bf16 rounding points); a dropped LoRA term gives 0.13


def _step_errors(w, c, hf, seed, T=21, BS=16):
    tokens = np.random.default_rng(100 + seed).integers(0, 96, T)
    with torch.no_grad():
        ref = hf(torch.from_numpy(tokens)[None]).logits[0].numpy().astype(np.float64)
    nb = 4
    kcs = [np.zeros((nb, c["n_kv"], BS, c["head_dim"]), np.uint16) for _ in range(2)]
    vcs = [np.zeros_like(k) for k in kcs]
    table = np.arange(nb, dtype=np.int32)[::-1].copy()[None, :]  # reversed physical order
    orc = Qwen2DecodeOracle(w, c)
    out = []
    for t in range(T):
        logits, nxt = orc.step(tokens[t:t + 1], kcs, vcs, table, np.array([t]))
        got = bf16_bits_to_f32(logits)[0].astype(np.float64)
        out.append((rel_err(got, ref[t]), int(nxt[0]), ref[t]))
    return out


@pytest.mark.parametrize("seed", [0, 1])
def test_decode_step_matches_transformers_qwen2(seed):
    w, c, hf = _tiny_model(seed)
    for t, (err, nxt, ref) in enumerate(_step_errors(w, c, hf, seed)):
        assert err <= TOL, t
        # the greedy token is the transformers argmax unless the top two are within tolerance
        top2 = np.sort(ref)[-2:]
        if top2[1] - top2[0] > TOL * np.abs(ref).max():
            assert nxt == np.argmax(ref), t


def test_planted_oracle_mistake_is_detected():
    """A plausible mistake in the oracle (the LoRA term dropped) fails the check."""
    w, c, hf = _tiny_model(0)
    bad = dict(c, scaling=0.0)
    assert max(e for e, _, _ in _step_errors(w, bad, hf, 0)) > 5 * TOL
