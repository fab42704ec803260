"""Pins the LLaMA-graph oracle (oracle/llama_oracle.py) on the CPU.

The forward pass is checked against HuggingFace transformers'
LlamaForCausalLM -- an independent implementation -- on the reference's own
toy_llama fixture (tests/testdata/toy_llama of the reference, copied to
tests/golden/toy_llama) and on a random grouped-query config; each operator
is checked against closed forms, numpy library routines and invariants
chosen so that a dropped term, a wrong sign or a transposed operand fails.
"""
from __future__ import annotations

import json
import math
import os

import numpy as np
import pytest

import llama_oracle as L
import oracle as Q

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "toy_llama")


def _toy():
    from safetensors.numpy import load_file

    tensors = load_file(os.path.join(GOLDEN, "model.safetensors"))
    cfg = L.LlamaConfig(vocab_size=256, hidden_size=64, intermediate_size=128, num_layers=2, num_heads=4,
                        num_kv_heads=4, rms_norm_eps=1e-5, rope_theta=10000.0, tie_word_embeddings=True)
    return cfg, tensors


def _hf_logits(cfg_dict: dict, tensors: dict, tokens) -> np.ndarray:
    torch = pytest.importorskip("torch")
    transformers = pytest.importorskip("transformers")
    hc = transformers.LlamaConfig(**cfg_dict)
    model = transformers.LlamaForCausalLM(hc).eval()
    res = model.load_state_dict({k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in tensors.items()},
                                strict=False)
    assert not res.missing_keys or res.missing_keys == ["lm_head.weight"], res
    with torch.no_grad():
        return model(torch.tensor([list(tokens)])).logits[0].float().numpy()


# ------------------------------------------------------------ forward pass

def test_toy_llama_prefill_matches_transformers():
    cfg, tensors = _toy()
    w = L.load_toy_llama(tensors, cfg)
    tokens = [1, 2, 3, 4, 5]          # the reference's toy prompt (test_tinyllama_e2e.cpp:67)
    ours, _ = L.prefill(cfg, w, tokens)
    with open(os.path.join(GOLDEN, "config.json")) as f:
        cfg_dict = {k: v for k, v in json.load(f).items() if k != "architectures"}
    ref = _hf_logits(cfg_dict, tensors, tokens)
    assert ours.shape == ref.shape == (5, 256)
    assert np.abs(ours - ref).max() <= 1e-5 * np.abs(ref).max()
    fused, _ = L.prefill(cfg, w, tokens, fused=True)
    assert np.abs(fused - ref).max() <= 1e-5 * np.abs(ref).max()


def test_gqa_config_matches_transformers():
    torch = pytest.importorskip("torch")
    transformers = pytest.importorskip("transformers")
    cfg_dict = dict(vocab_size=96, hidden_size=64, intermediate_size=80, num_hidden_layers=2, num_attention_heads=8,
                    num_key_value_heads=2, rms_norm_eps=1e-6, rope_theta=500.0, max_position_embeddings=64,
                    tie_word_embeddings=False)
    torch.manual_seed(7)
    model = transformers.LlamaForCausalLM(transformers.LlamaConfig(**cfg_dict)).eval()
    with torch.no_grad():  # non-trivial norm weights, so a dropped weight term shows
        for name, p in model.named_parameters():
            if name.endswith("norm.weight"):
                p.uniform_(0.5, 1.5)
    tensors = {k: v.detach().float().numpy().copy() for k, v in model.state_dict().items()}
    tokens = [3, 17, 94, 0, 55, 21, 8]
    with torch.no_grad():
        ref = model(torch.tensor([tokens])).logits[0].float().numpy()
    cfg = L.LlamaConfig(vocab_size=96, hidden_size=64, intermediate_size=80, num_layers=2, num_heads=8,
                        num_kv_heads=2, rms_norm_eps=1e-6, rope_theta=500.0)
    w = L.load_toy_llama(tensors, cfg)
    for fused in (False, True):
        ours, _ = L.prefill(cfg, w, tokens, fused=fused)
        assert np.abs(ours - ref).max() <= 2e-5 * np.abs(ref).max(), fused


def test_decode_after_prefill_equals_longer_prefill():
    cfg, tensors = _toy()
    w = L.load_toy_llama(tensors, cfg)
    prompt = [1, 10, 20, 30, 40, 50]
    full, _ = L.prefill(cfg, w, prompt)
    for fused in (False, True):
        _, kv = L.prefill(cfg, w, prompt[:3], fused=fused)
        for pos in range(3, 6):
            step = L.decode(cfg, w, prompt[pos], pos, kv, fused=fused)
            assert np.abs(step[0] - full[pos]).max() <= 1e-5 * np.abs(full).max()
        assert kv["k"][0].shape == (4, 6, 16)


def test_int8_quantized_toy_llama_quality():
    # The reference's own acceptance test (tests/test_quantization.cpp:480-545):
    # INT8 per-channel linears, prompt {1, 10, 20, 30}, last-token logits.
    cfg, tensors = _toy()
    w = L.load_toy_llama(tensors, cfg)
    ref, _ = L.prefill(cfg, w, [1, 10, 20, 30], last_only=True)
    qw = L.quantize_linears(w, Q.QUANT_INT8, 0)
    out, _ = L.prefill(cfg, qw, [1, 10, 20, 30], last_only=True)
    _, rmse, _, cosine = Q.metrics(ref[0], out[0])
    assert cosine > 0.999 and rmse < 0.15
    assert int(np.argmax(ref)) == int(np.argmax(out))


# -------------------------------------------------------------- operators

def test_rope_identity_norm_and_composition():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 5, 16)).astype(np.float32)
    c0, s0 = L.rope_cache(1, 16, 10000.0, 0)
    assert np.array_equal(L.rope(x, c0, s0), x)                    # position 0
    c, s = L.rope_cache(5, 16, 10000.0, 7)
    y = L.rope(x, c, s)
    pair = lambda t: t[..., :8] ** 2 + t[..., 8:] ** 2           # noqa: E731
    assert np.allclose(pair(y), pair(x), rtol=1e-5, atol=1e-6)
    ca, sa = L.rope_cache(1, 16, 10000.0, 3)
    cb, sb = L.rope_cache(1, 16, 10000.0, 4)
    cab, sab = L.rope_cache(1, 16, 10000.0, 7)
    two = L.rope(L.rope(x, ca, sa), cb, sb)
    assert np.allclose(two, L.rope(x, cab, sab), atol=1e-5)
    # head_dim 2 at position p: a plain 2-D rotation by angle p.
    c2, s2 = L.rope_cache(1, 2, 10000.0, 3)
    v = np.array([[1.0, 2.0]], np.float32)
    r = L.rope(v, c2, s2)[0]
    assert np.allclose(r, [math.cos(3) - 2 * math.sin(3), 2 * math.cos(3) + math.sin(3)], atol=1e-6)


def test_rope_positions_follow_rows_of_cache():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((2, 4, 8)).astype(np.float32)   # [H, S, D]
    c, s = L.rope_cache(4, 8, 100.0, 0)
    y = L.rope(x, c, s)
    for t in range(4):
        ct, st = L.rope_cache(1, 8, 100.0, t)
        assert np.allclose(y[:, t], L.rope(x[:, t], ct, st), atol=1e-6)


def test_rmsnorm_closed_forms():
    x = np.array([[3.0, 4.0]], np.float32)
    y = L.rmsnorm(x, np.ones(2, np.float32), 1e-5)
    assert np.allclose(y, x / math.sqrt(12.5 + 1e-5), rtol=1e-6)
    rng = np.random.default_rng(3)
    x = rng.standard_normal((6, 32)).astype(np.float32)
    y = L.rmsnorm(x, np.ones(32, np.float32), 1e-12)
    assert np.allclose(np.sqrt((y.astype(np.float64) ** 2).mean(-1)), 1.0, atol=1e-5)
    w = rng.uniform(0.5, 2, 32).astype(np.float32)
    assert np.allclose(L.rmsnorm(5 * x, w, 1e-12), L.rmsnorm(x, w, 1e-12), rtol=1e-5, atol=1e-6)
    assert np.allclose(L.rmsnorm(x, w, 1e-12), y * w, rtol=1e-6, atol=1e-7)


def test_softmax_closed_forms():
    a = np.array([[0.3, -1.2], [5.0, 5.0]], np.float32)
    y = L.softmax(a)
    assert np.allclose(y[:, 0], 1 / (1 + np.exp(a[:, 1] - a[:, 0])), rtol=1e-6)
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 7, 5)).astype(np.float32)
    for ax in (0, 1, 2, -1):
        y = L.softmax(x, ax)
        assert np.allclose(y.sum(axis=ax), 1.0, atol=1e-6)
        assert np.allclose(L.softmax(x + 10.0, ax), y, atol=1e-6)


def test_attention_special_cases():
    rng = np.random.default_rng(5)
    q = rng.standard_normal((1, 2, 3, 8)).astype(np.float32)
    k = rng.standard_normal((1, 2, 1, 8)).astype(np.float32)
    v = rng.standard_normal((1, 2, 1, 6)).astype(np.float32)
    out = L.attention(q, k, v, 0.0, False)                       # one key -> its value
    assert np.allclose(out, np.broadcast_to(v, out.shape), atol=1e-6)
    kz = np.zeros((1, 2, 4, 8), np.float32)                       # equal scores -> mean of values
    v4 = rng.standard_normal((1, 2, 4, 6)).astype(np.float32)
    assert np.allclose(L.attention(q, kz, v4, 0.0, False), v4.mean(axis=2, keepdims=True), atol=1e-6)


def test_attention_gqa_and_causal_structure():
    rng = np.random.default_rng(6)
    q = rng.standard_normal((2, 8, 3, 16)).astype(np.float32)
    k = rng.standard_normal((2, 2, 5, 16)).astype(np.float32)
    v = rng.standard_normal((2, 2, 5, 12)).astype(np.float32)
    gqa = L.attention(q, k, v, 0.5, True)
    mha = L.attention(q, L.repeat_kv(k, 4, 1), L.repeat_kv(v, 4, 1), 0.5, True)
    assert np.array_equal(gqa, mha)
    for i in range(3):  # causal row i == non-causal attention over its visible keys 0..5-3+i
        n = 5 - 3 + i + 1
        row = L.attention(q[:, :, i:i + 1], k[:, :, :n], v[:, :, :n], 0.5, False)
        assert np.allclose(gqa[:, :, i:i + 1], row, atol=1e-6)
    s = (q[0, 0] @ k[0, 0].T) * 0.5                                # explicit softmax(QK^T)V for one head
    p = np.exp(s - s.max(-1, keepdims=True))
    mask = np.arange(5)[None, :] <= np.arange(3)[:, None] + 2
    p = np.where(mask, p, 0)
    assert np.allclose(gqa[0, 0], (p / p.sum(-1, keepdims=True)) @ v[0, 0], atol=1e-5)
    # Sq > Sk is rejected by the signature when causal; rows with no key are zero.
    z = L.attention(q[:, :, :3], k[:, :, :1], v[:, :, :1], 1.0, True)
    assert np.all(z[:, :, :2] == 0)


def test_layout_ops_against_numpy():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((3, 4, 5)).astype(np.float32)
    assert np.array_equal(L.transpose(x, (1, 0, 2)), x.transpose(1, 0, 2))
    assert np.array_equal(L.transpose(x, ()), x.transpose(2, 1, 0))     # empty perm reverses
    assert np.array_equal(L.slice_(x, [-1], [3]), x[2:3])
    assert np.array_equal(L.slice_(x, [0, 1], [3, 100], [2, 2]), x[0:3:2, 1:4:2])
    assert L.slice_(x, [2], [1]).shape == (0, 4, 5)
    assert np.array_equal(L.concat(x, x[:, :2], 1), np.concatenate([x, x[:, :2]], 1))
    r = L.repeat_kv(x, 3, 0)
    assert r.shape == (9, 4, 5) and all(np.array_equal(r[h], x[h // 3]) for h in range(9))
    idx = np.array([[2, 0], [1, 1]], np.int32)
    assert np.array_equal(L.embedding(x[0], idx), x[0][idx])
    with pytest.raises(IndexError):
        L.embedding(x[0], np.array([4], np.int32))


# ------------------------------------------- linear modes (exact, dense)

def _packed_linear(rng, k, n, qt, mode):
    w = (rng.standard_normal((k, n)) * 0.02).astype(np.float32)
    if qt == Q.QUANT_INT8:
        q, s = Q.quantize_int8(w)
        return L.Linear(q=q, s=s, k=k, n=n, quant_type=qt, block=0, mode=mode)
    q, s = Q.quantize_int4(w, 32)
    return L.Linear(q=q, s=s, k=k, n=n, quant_type=qt, block=32, mode=mode)


def test_dense_blockwise_int8_matches_the_scalar_oracle():
    # INT8 codes with block scales (QuantizedMatMulAttrs.block_size > 0)
    rng = np.random.default_rng(3)
    k, n, block = 100, 24, 32
    q = rng.integers(-127, 128, (k, n), dtype=np.int8)
    s = (rng.random((-(-k // block), n)) * 10.0 ** rng.uniform(-3, 1, (-(-k // block), n))).astype(np.float32)
    lin = L.Linear(q=q, s=s, k=k, n=n, quant_type=Q.QUANT_INT8, block=block, mode=L.LINEAR_EXACT)
    x = rng.standard_normal((5, k)).astype(np.float32)
    exact = lin(x)
    lin.mode = L.LINEAR_DENSE
    assert np.abs(lin(x) - exact).max() <= 1e-5 * np.abs(exact).max()


@pytest.mark.parametrize("qt", [Q.QUANT_INT8, Q.QUANT_INT4])
@pytest.mark.parametrize("m", [1, 3, 9])
def test_dense_mode_matches_the_scalar_oracle(qt, m):
    rng = np.random.default_rng(7 + m)
    k, n = 96, 48
    lin = _packed_linear(rng, k, n, qt, L.LINEAR_EXACT)
    x = rng.standard_normal((m, k)).astype(np.float32)
    exact = lin(x)
    lin.mode = L.LINEAR_DENSE
    dense = lin(x)
    assert np.abs(dense - exact).max() <= 1e-5 * np.abs(exact).max()


def test_codes_unpack_to_the_dequantized_weights():
    rng = np.random.default_rng(3)
    for qt in (Q.QUANT_INT8, Q.QUANT_INT4):
        lin = _packed_linear(rng, 70, 32, qt, L.LINEAR_DENSE)
        c = lin.codes().astype(np.float32)
        assert c.shape == (70, 32) and np.abs(c).max() <= (127 if qt == Q.QUANT_INT8 else 7)
        scale = lin.s.reshape(-1, 32)
        per_row = scale if qt == Q.QUANT_INT8 else np.repeat(scale, 32, axis=0)[:70]
        assert np.array_equal(c * per_row, lin.dense())


def test_split_rows_fp16_closed_forms():
    # a tie of hi (1 + 2^-11 between 1 and 1 + 2^-10) is carried by lo
    tie = np.float32(1 + 2.0 ** -11)
    r = L.split_rows_fp16(np.array([[1.75, tie, -tie]], np.float32))
    assert r.tolist() == [[1.75, float(tie), -float(tie)]]
    # large rows: 1e6 = 999936 (hi) + 64 (lo); no overflow
    r = L.split_rows_fp16(np.array([[1e6, 3.0, -2.5e5], [1e30, -7e29, 1.0]], np.float32))
    assert r[0].tolist() == [1e6, 3.0, -2.5e5]
    assert r[1, :2].tolist() == [float(np.float32(1e30)), float(np.float32(-7e29))]
    assert r[1, 2] == 0.0      # 1e-30 of its row's maximum: below fp16's subnormals after scaling
    # 22 significant bits: an element needing 24 loses at most 2^-23 of itself
    x = np.array([[1.0, 1 + 2.0 ** -11 - 2.0 ** -23, 1 + 2.0 ** -23]], np.float32)
    r = L.split_rows_fp16(x)
    assert r[0, 1] == 1 + 2.0 ** -11 and r[0, 2] == 1 + 2.0 ** -23
    rng = np.random.default_rng(2)
    y = (rng.standard_normal((4, 512)) * 10.0 ** rng.uniform(-6, 6, (4, 512))).astype(np.float32)
    ry = L.split_rows_fp16(y)
    rowmax = np.abs(y).max(axis=1, keepdims=True).astype(np.float64)
    assert np.all(np.abs(ry - y) <= np.maximum(2.0 ** -22 * np.abs(y), 2.0 ** -37 * rowmax))
    # all-zero rows stay zero; a row holding an infinity is not scaled
    r = L.split_rows_fp16(np.array([[0.0, 0.0], [np.inf, 1.0]], np.float32))
    assert r[0].tolist() == [0.0, 0.0] and r[1, 0] == np.inf and r[1, 1] == 1.0


def test_load_packed_reads_the_packed_layout():
    rng = np.random.default_rng(5)
    cfg = L.LlamaConfig(vocab_size=40, hidden_size=64, intermediate_size=96, num_layers=2, num_heads=4,
                        num_kv_heads=2)
    d = cfg.head_dim
    shapes = {"self_attn.q_proj": (64, 64), "self_attn.k_proj": (64, 2 * d), "self_attn.v_proj": (64, 2 * d),
              "self_attn.o_proj": (64, 64), "mlp.gate_proj": (64, 96), "mlp.up_proj": (64, 96),
              "mlp.down_proj": (96, 64)}
    tensors, ref = {}, {}
    for layer in range(2):
        for hf, (k, n) in shapes.items():
            q, s = Q.quantize_int4((rng.standard_normal((k, n)) * 0.02).astype(np.float32), 32)
            name = f"model.layers.{layer}.{hf}.weight"
            tensors[name + ".codes"], tensors[name + ".scales"] = q.view(np.int8), s
            ref[name] = (q, s)
        tensors[f"model.layers.{layer}.input_layernorm.weight"] = np.ones(64, np.float32)
        tensors[f"model.layers.{layer}.post_attention_layernorm.weight"] = np.ones(64, np.float32)
    q, s = Q.quantize_int4((rng.standard_normal((64, 40)) * 0.02).astype(np.float32), 32)
    tensors["lm_head.weight.codes"], tensors["lm_head.weight.scales"] = q.view(np.int8), s
    tensors["model.embed_tokens.weight"] = rng.standard_normal((40, 64)).astype(np.float32)
    tensors["model.norm.weight"] = np.ones(64, np.float32)
    w = L.load_packed(tensors, cfg, Q.QUANT_INT4, 32)
    assert w.down[1].k == 96 and w.down[1].n == 64 and w.wk[0].n == 2 * d
    assert np.array_equal(w.gate[1].q.view(np.uint8), ref["model.layers.1.mlp.gate_proj.weight"][0])
    # the model runs in every linear mode and they agree
    logits_exact, _ = L.prefill(cfg, w, [3, 1, 4, 1, 5, 9], last_only=True)
    L.set_linear_mode(w, L.LINEAR_DENSE)
    logits_dense, _ = L.prefill(cfg, w, [3, 1, 4, 1, 5, 9], last_only=True)
    assert np.abs(logits_dense - logits_exact).max() <= 1e-5 * np.abs(logits_exact).max()
