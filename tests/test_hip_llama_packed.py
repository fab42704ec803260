"""Pre-packed LLaMA weights (velomind/llama/llama_packed.h, C ABI in
include/vm_llama.h): every linear packed once on the GPU, written to a
safetensors file of I8 codes and F32 scales, read back and run by the
resident decoder without packing.

Checks:
  * the file, read with the Hugging Face safetensors library (not our
    reader), holds for every linear the oracle's quant.cpp packing of the
    same fp32 weights byte for byte (quant.cpp:74-175), the embedding and
    norms unchanged, and the model config in its metadata;
  * a session from the loaded file gives logits and greedy tokens identical
    to a session that packs the same fp32 weights itself (same packed bytes,
    same kernels), and the greedy tokens of the oracle's quantized model;
  * a config that differs from the file's, a file that is not a packed
    file, and a missing file are refused with an error.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

import llama_oracle as L
import oracle as Q

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "toy_llama")


@pytest.fixture(scope="module")
def llama(hip):
    from velomind_hip import llama as VL

    return VL


def _gqa(seed):
    cfg = L.LlamaConfig(vocab_size=300, hidden_size=512, intermediate_size=384, num_layers=2, num_heads=8,
                        num_kv_heads=2, rms_norm_eps=1e-5, rope_theta=10000.0)
    rng = np.random.default_rng(seed)
    n = lambda *s: (rng.standard_normal(s) * 0.05).astype(np.float32)  # noqa: E731
    lin = lambda k, m: L._lin(n(k, m))                                   # noqa: E731
    h, kv, i = cfg.hidden_size, cfg.kv_heads * cfg.head_dim, cfg.intermediate_size
    w = L.LlamaWeights(embed=n(cfg.vocab_size, h) * 10, final_norm=1 + n(h), lm_head=lin(h, cfg.vocab_size))
    for _ in range(cfg.num_layers):
        w.attn_norm.append(1 + n(h))
        w.ffn_norm.append(1 + n(h))
        w.wq.append(lin(h, h))
        w.wk.append(lin(h, kv))
        w.wv.append(lin(h, kv))
        w.wo.append(lin(h, h))
        w.gate.append(lin(h, i))
        w.up.append(lin(h, i))
        w.down.append(lin(i, h))
    return cfg, w


_LINEARS = (("wq", "self_attn.q_proj"), ("wk", "self_attn.k_proj"), ("wv", "self_attn.v_proj"),
            ("wo", "self_attn.o_proj"), ("gate", "mlp.gate_proj"), ("up", "mlp.up_proj"), ("down", "mlp.down_proj"))


def _check_file(path, cfg, w, qt, block):
    from safetensors.numpy import load_file
    from safetensors import safe_open

    with safe_open(path, framework="numpy") as f:
        meta = f.metadata()
    assert meta["velomind.format"] == "packed-linear-v1"
    assert meta["velomind.quant_type"] == ("int4" if qt == Q.QUANT_INT4 else "int8")
    assert int(meta["velomind.block_size"]) == block
    for key in ("vocab_size", "hidden_size", "intermediate_size", "num_layers", "num_heads"):
        assert int(meta["velomind." + key]) == getattr(cfg, key), key
    assert int(meta["velomind.num_kv_heads"]) == cfg.kv_heads
    assert np.float32(meta["velomind.rms_norm_eps"]) == np.float32(cfg.rms_norm_eps)
    assert np.float32(meta["velomind.rope_theta"]) == np.float32(cfg.rope_theta)

    t = load_file(path)
    assert len(t) == 2 * (7 * cfg.num_layers + 1) + 2 + 2 * cfg.num_layers

    def expect(name, lin):
        if qt == Q.QUANT_INT4:
            q, s = Q.quantize_int4(lin.w, block)
        else:
            q, s = Q.quantize_int8(lin.w)
        codes, scales = t[name + ".codes"], t[name + ".scales"]
        assert codes.dtype == np.int8 and scales.dtype == np.float32, name
        assert codes.shape == q.shape and scales.shape == s.shape, name
        assert np.array_equal(codes.view(np.uint8), q.view(np.uint8)), f"{name}: codes differ from quant.cpp"
        assert np.array_equal(scales.view(np.uint32), s.view(np.uint32)), f"{name}: scales differ from quant.cpp"

    assert np.array_equal(t["model.embed_tokens.weight"], w.embed)
    assert np.array_equal(t["model.norm.weight"], w.final_norm)
    expect("lm_head.weight", w.lm_head)
    for layer in range(cfg.num_layers):
        p = f"model.layers.{layer}."
        assert np.array_equal(t[p + "input_layernorm.weight"], w.attn_norm[layer])
        assert np.array_equal(t[p + "post_attention_layernorm.weight"], w.ffn_norm[layer])
        for attr, hf in _LINEARS:
            expect(p + hf + ".weight", getattr(w, attr)[layer])


@pytest.mark.parametrize("qt,block", [(Q.QUANT_INT8, 0), (Q.QUANT_INT4, 32), (Q.QUANT_INT4, 64)])
def test_packed_file_matches_oracle_and_runs(llama, tmp_path, qt, block):
    cfg, w = _gqa(seed=21 + block)
    print(f"case packed gqa qt={qt} block={block}", flush=True)
    dev = llama.Weights.from_oracle(cfg, w)
    path = str(tmp_path / "packed.safetensors")
    packed = llama.PackedWeights.pack(dev, qt, block)
    packed.save(path)
    packed.close()
    _check_file(path, cfg, w, qt, block)

    fc = llama.PackedWeights.file_config(path)
    assert (fc.vocab_size, fc.hidden_size, fc.num_layers, fc.num_kv_heads) == (300, 512, 2, 2)
    loaded = llama.PackedWeights.load(path)          # config from the file
    s_file = llama.Session.from_packed(loaded, max_seq=64)
    loaded.close()                                    # the session keeps its own copy
    s_pack = llama.Session(dev, llama.ENGINE_RESIDENT, qt, block, max_seq=64)

    prompt = [3, 1, 4]
    assert np.array_equal(s_file.prefill(prompt), s_pack.prefill(prompt))
    for pos, tok in ((3, 1), (4, 5)):
        assert np.array_equal(s_file.forward_step(tok, pos), s_pack.forward_step(tok, pos)), pos
    long_prompt = list(range(7, 7 + 70, 3))[:19]
    assert np.array_equal(s_file.prefill(long_prompt), s_pack.prefill(long_prompt))

    ow = L.quantize_linears(w, qt, block)
    ref_tokens, _ = L.greedy(cfg, ow, [2, 7, 1], 6)
    a, _ = s_file.generate([2, 7, 1], 6, use_hip_graph=True)
    b, _ = s_pack.generate([2, 7, 1], 6, use_hip_graph=True)
    assert list(a) == list(b) == ref_tokens


def test_packed_toy_llama_file_matches_oracle(llama, tmp_path):
    """The toy_llama fixture (head_dim 16, which the resident decoder does
    not run): packing and the file format alone."""
    from safetensors.numpy import load_file

    cfg = L.LlamaConfig(vocab_size=256, hidden_size=64, intermediate_size=128, num_layers=2, num_heads=4,
                        num_kv_heads=4, rms_norm_eps=1e-5, rope_theta=10000.0)
    w = L.load_toy_llama(load_file(os.path.join(GOLDEN, "model.safetensors")), cfg)
    print("case packed toy_llama int4", flush=True)
    path = str(tmp_path / "toy.safetensors")
    p = llama.PackedWeights.pack(llama.Weights.from_oracle(cfg, w), Q.QUANT_INT4, 32)
    p.save(path)
    _check_file(path, cfg, w, Q.QUANT_INT4, 32)
    with pytest.raises(RuntimeError, match="head_dim"):
        llama.Session.from_packed(p, max_seq=16)


def test_packed_load_errors(llama, tmp_path):
    cfg, w = _gqa(seed=2)
    print("case packed errors", flush=True)
    path = str(tmp_path / "p.safetensors")
    llama.PackedWeights.pack(llama.Weights.from_oracle(cfg, w), Q.QUANT_INT8, 0).save(path)
    wrong = L.LlamaConfig(vocab_size=300, hidden_size=512, intermediate_size=384, num_layers=3, num_heads=8,
                          num_kv_heads=2, rms_norm_eps=1e-5, rope_theta=10000.0)
    with pytest.raises(RuntimeError, match="config"):
        llama.PackedWeights.load(path, wrong)
    with pytest.raises(RuntimeError, match="packed-linear-v1"):
        llama.PackedWeights.load(os.path.join(GOLDEN, "model.safetensors"))
    with pytest.raises(RuntimeError, match="cannot read"):
        llama.PackedWeights.load(str(tmp_path / "missing.safetensors"), cfg)
    with pytest.raises(RuntimeError):
        llama.PackedWeights.pack(llama.Weights.from_oracle(cfg, w), Q.QUANT_INT8, 32)   # INT8 is per column
