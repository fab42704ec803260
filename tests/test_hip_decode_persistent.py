"""The one-launch decode step (vm_hip_decode_step, the resident decoder's
one-token step under VELOMIND_DECODE_PERSISTENT=1) against the oracle and
against the default launch-per-projection step.

Covers INT8 per column and INT4 block 32, grouped-query attention, decode
positions that cross the 32-key attention chunks, greedy generation, and a
context long enough that the attention items outnumber the workgroups (each
workgroup then takes several).  Bound: 1e-4 of max |logit| against the
oracle (LINEAR_DENSE mode; decode steps are fp32 GEMVs), 1e-5 against the
other step (the same arithmetic, summed in another grouping).
"""
from __future__ import annotations

import numpy as np
import pytest

import llama_oracle as L

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def llama(hip):
    from velomind_hip import llama as VL

    return VL


def _close(out, ref, rel, what):
    out = np.asarray(out, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    err = np.abs(out - ref).max()
    assert err <= rel * np.abs(ref).max(), f"{what}: max abs err {err:.3e} > {rel * np.abs(ref).max():.3e}"


def _model(seed, hidden, heads, kv_heads, inter, vocab, layers, scale=0.05):
    cfg = L.LlamaConfig(vocab_size=vocab, hidden_size=hidden, intermediate_size=inter, num_layers=layers,
                        num_heads=heads, num_kv_heads=kv_heads, rms_norm_eps=1e-5, rope_theta=10000.0)
    rng = np.random.default_rng(seed)
    n = lambda *s: (rng.standard_normal(s) * scale).astype(np.float32)  # noqa: E731
    lin = lambda k, m: L._lin(n(k, m))                                   # noqa: E731
    kv = kv_heads * cfg.head_dim
    w = L.LlamaWeights(embed=n(vocab, hidden) * 10, final_norm=1 + n(hidden), lm_head=lin(hidden, vocab))
    for _ in range(layers):
        w.attn_norm.append(1 + n(hidden))
        w.ffn_norm.append(1 + n(hidden))
        w.wq.append(lin(hidden, hidden))
        w.wk.append(lin(hidden, kv))
        w.wv.append(lin(hidden, kv))
        w.wo.append(lin(hidden, hidden))
        w.gate.append(lin(hidden, inter))
        w.up.append(lin(hidden, inter))
        w.down.append(lin(inter, hidden))
    return cfg, w


def _sessions(llama, monkeypatch, dev, qt, block, max_seq):
    monkeypatch.setenv("VELOMIND_DECODE_PERSISTENT", "1")
    sp = llama.Session(dev, llama.ENGINE_RESIDENT, qt, block, max_seq=max_seq)
    monkeypatch.setenv("VELOMIND_DECODE_PERSISTENT", "0")
    ss = llama.Session(dev, llama.ENGINE_RESIDENT, qt, block, max_seq=max_seq)
    monkeypatch.delenv("VELOMIND_DECODE_PERSISTENT")
    assert sp.decode_path() == llama.DECODE_PERSISTENT
    assert ss.decode_path() in (llama.DECODE_SLICES, llama.DECODE_PER_OP)
    return sp, ss


@pytest.mark.parametrize("qt,block", [(1, 0), (2, 32)])
def test_persistent_step_matches_oracle_and_slices(llama, monkeypatch, qt, block):
    cfg, w = _model(11, hidden=512, heads=8, kv_heads=2, inter=384, vocab=320, layers=2)
    ow = L.set_linear_mode(L.quantize_linears(w, qt, block), L.LINEAR_DENSE)
    dev = llama.Weights.from_oracle(cfg, w)
    sp, ss = _sessions(llama, monkeypatch, dev, qt, block, max_seq=80)
    prompt = [3, 1, 4]
    ref, kv = L.prefill(cfg, ow, prompt, last_only=True)
    _close(sp.prefill(prompt), ref[0], 1e-4, "prefill")
    ss.prefill(prompt)
    rng = np.random.default_rng(7)
    toks = rng.integers(0, cfg.vocab_size, 70)
    # positions 3 .. 72: the 32-key chunks fill and a second and third start
    for pos in range(3, 73):
        tok = int(toks[pos - 3])
        print(f"case persistent qt={qt} pos={pos}", flush=True)
        zp = sp.forward_step(tok, pos)
        zs = ss.forward_step(tok, pos)
        zr = L.decode(cfg, ow, tok, pos, kv)[0]
        if pos in (3, 4, 31, 32, 33, 63, 64, 65, 72):
            _close(zp, zr, 1e-4, f"pos {pos} vs oracle")
        _close(zp, zs, 1e-5, f"pos {pos} vs slices")


@pytest.mark.parametrize("qt,block", [(1, 0), (2, 32)])
def test_persistent_generate_is_greedy(llama, monkeypatch, qt, block):
    cfg, w = _model(5, hidden=512, heads=8, kv_heads=2, inter=384, vocab=320, layers=2)
    ow = L.set_linear_mode(L.quantize_linears(w, qt, block), L.LINEAR_DENSE)
    dev = llama.Weights.from_oracle(cfg, w)
    sp, ss = _sessions(llama, monkeypatch, dev, qt, block, max_seq=64)
    prompt = [2, 7, 1, 8, 2, 8]
    ref_tokens, _ = L.greedy(cfg, ow, prompt, 24)
    print(f"case persistent generate qt={qt}", flush=True)
    a, _ = sp.generate(prompt, 24)
    b, _ = ss.generate(prompt, 24)
    c, _ = sp.generate(prompt, 24)     # again on the same workspace
    assert list(a) == list(b) == list(c) == ref_tokens


def test_persistent_long_context_several_items_per_workgroup(llama, monkeypatch):
    # 8 KV heads x 33 key chunks at position 1040: more attention items than
    # the 256 workgroups of an MI355X
    cfg, w = _model(3, hidden=512, heads=8, kv_heads=8, inter=256, vocab=256, layers=1)
    ow = L.set_linear_mode(L.quantize_linears(w, 2, 32), L.LINEAR_DENSE)
    dev = llama.Weights.from_oracle(cfg, w)
    sp, ss = _sessions(llama, monkeypatch, dev, 2, 32, max_seq=1100)
    prompt = list(np.random.default_rng(4).integers(0, cfg.vocab_size, 1040))
    print("case persistent long context", flush=True)
    ref, kv = L.prefill(cfg, ow, prompt, last_only=True)
    sp.prefill(prompt)
    ss.prefill(prompt)
    for pos, tok in ((1040, 17), (1041, 200), (1042, 5)):
        zp = sp.forward_step(tok, pos)
        _close(zp, ss.forward_step(tok, pos), 1e-5, f"pos {pos} vs slices")
        _close(zp, L.decode(cfg, ow, tok, pos, kv)[0], 1e-4, f"pos {pos} vs oracle")
