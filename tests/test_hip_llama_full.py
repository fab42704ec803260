"""BASELINE configs 4 and 5 end to end at full size, against the oracle.

  config 5  TinyLlama-1.1B shapes (22 layers, hidden 2048, 32 / 4 heads,
            intermediate 5632, vocab 32000, RoPE theta 1e4), INT4 block 32,
            a 512-token uniform-random prompt
  config 4  SmolLM2-360M shapes (32 layers, hidden 960, 15 / 5 heads,
            intermediate 2560, vocab 49152, RoPE theta 1e5, tied
            embeddings), INT8 per column, a 128-token prompt

Weights are synthetic N(0, 0.02) (norms N(1, 0.02)), generated and packed
on the GPU, saved as a pre-packed safetensors file and read back with the
safetensors library: the oracle (oracle/llama_oracle.py) runs on exactly
those codes and scales, in its LINEAR_DENSE mode (the dequantized weights
times x in fp32, the reference QuantizedMatMul's sum in another order,
pinned against LINEAR_EXACT in tests/test_oracle_llama.py).

Tolerance.  At these depths the synthetic networks amplify fp32 rounding:
perturbing the oracle's embedding by 2^-24 relative noise moves its
TinyLlama logits by ~6e-4 of max|logit| at 512 tokens (SmolLM2: ~3e-5).
No implementation in fp32 can be held closer to the oracle than that, so
each comparison is held to TOL_FACTOR times the spread the oracle itself
shows under two such perturbations (never below 1e-4 of max|logit|), plus
the reference's own end-to-end criteria, cosine > 0.999 and the same
argmax (tests/test_quantization.cpp:480-546).

Late positions: the bench decodes TinyLlama at positions 512..767 and
SmolLM2 at 128..255; a prompt that ends LATE_STEPS positions before the
last, followed by LATE_STEPS teacher-forced decode steps on the resident
decoder (the kernels of the bench's decode step, with its max_seq),
reaches the same last positions, and each step's logits are held to the
oracle as above.

Reference arithmetic: the prompt logits are also compared with the oracle
in its LINEAR_EXACT mode (the reference CPU QuantizedMatMul's own loop,
exact codes and scales) under the reference's end-to-end criteria, cosine >
0.999, rmse < 0.15 and the same argmax (tests/test_quantization.cpp:537-545).

Both engines are checked: the resident decoder, and the graph engine (the
reference engine's loop, a Graph on DeviceType::HIP per call,
llama_engine.cpp:333-455), each for
  * the last-position prompt logits;
  * the first LOGIT_STEPS decode steps' logits;
  * STEPS greedy tokens, teacher-forced on the GPU's tokens: at each step the
    GPU's token is the oracle's argmax, or within the step's bound of it (a
    near-tie the bound cannot resolve).
"""
from __future__ import annotations

import numpy as np
import pytest

import llama_oracle as L
import oracle as Q

pytestmark = pytest.mark.gpu

FLOOR = 1e-4
TOL_FACTOR = 4.0
PERTURB = 2.0 ** -24
STEPS = 16
LOGIT_STEPS = 3
LATE_STEPS = 8

MODELS = {
    "tinyllama_1.1b_int4": dict(
        cfg=L.LlamaConfig(vocab_size=32000, hidden_size=2048, intermediate_size=5632, num_layers=22, num_heads=32,
                          num_kv_heads=4, rms_norm_eps=1e-5, rope_theta=10000.0),
        quant=2, block=32, prompt=512, decode=256, tied=False, seed=20240601),
    "smollm2_360m_int8": dict(
        cfg=L.LlamaConfig(vocab_size=49152, hidden_size=960, intermediate_size=2560, num_layers=32, num_heads=15,
                          num_kv_heads=5, rms_norm_eps=1e-5, rope_theta=100000.0, tie_word_embeddings=True),
        quant=1, block=0, prompt=128, decode=128, tied=True, seed=20240602),
}


def _rel(a, b) -> float:
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.abs(a - b).max() / np.abs(b).max())


def _close(out, ref, rel, what):
    out = np.asarray(out, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    got = _rel(out, ref)
    print(f"  {what}: max abs err {got:.2e} of max|logit| (bound {rel:.2e})", flush=True)
    assert got <= rel, f"{what}: max abs err {got:.3e} of max|logit| > {rel:.3e}"
    cos = float(out @ ref / (np.linalg.norm(out) * np.linalg.norm(ref)))
    assert cos > 0.999, f"{what}: cosine {cos}"


class OracleRun:
    """One oracle model state: the prompt's logits and KV cache, and
    teacher-forced decode logits cached per token prefix."""

    def __init__(self, cfg, w, prompt):
        self.cfg, self.w, self.n = cfg, w, len(prompt)
        logits, self.kv = L.prefill(cfg, w, prompt, last_only=True)
        self.logits = logits[0]
        self.cache = {}

    def decode(self, tokens):
        kv = {"k": list(self.kv["k"]), "v": list(self.kv["v"])}
        out = []
        for i, tok in enumerate(tokens):
            key = tuple(int(t) for t in tokens[: i + 1])
            if key not in self.cache:
                z = L.decode(self.cfg, self.w, int(tok), self.n + i, kv)[0]
                self.cache[key] = (z, {"k": list(kv["k"]), "v": list(kv["v"])})
            z, after = self.cache[key]
            kv = {"k": list(after["k"]), "v": list(after["v"])}
            out.append(z)
        return out


def _perturbed(w, seed):
    rng = np.random.default_rng(seed)
    e = w.embed
    noisy = (e.astype(np.float64) * (1 + PERTURB * rng.standard_normal(e.shape))).astype(np.float32)
    return L.LlamaWeights(embed=noisy, final_norm=w.final_norm, lm_head=w.lm_head, attn_norm=w.attn_norm,
                          ffn_norm=w.ffn_norm, wq=w.wq, wk=w.wk, wv=w.wv, wo=w.wo, gate=w.gate, up=w.up,
                          down=w.down)


@pytest.fixture(scope="module", params=list(MODELS))
def model(request, hip, tmp_path_factory):
    from safetensors.numpy import load_file
    from velomind_hip import llama as VL

    name = request.param
    spec = MODELS[name]
    cfg = spec["cfg"]
    print(f"\ncase {name}: weights on the GPU, packed, saved", flush=True)
    dev = VL.Weights(cfg)
    dev.fill_synthetic(spec["seed"], 0.02)
    if spec["tied"]:
        dev.tie_lm_head()
    packed = VL.PackedWeights.pack(dev, spec["quant"], spec["block"])
    path = tmp_path_factory.mktemp(name) / "packed.safetensors"
    packed.save(str(path))
    packed.close()
    ow = L.set_linear_mode(L.load_packed(load_file(str(path)), cfg, spec["quant"], spec["block"]), L.LINEAR_DENSE)
    path.unlink()
    if spec["tied"]:
        # the tie is real: the packed lm_head is quant.cpp's INT8 packing of
        # the embedding's transpose
        q, sc = Q.quantize_int8(np.ascontiguousarray(ow.embed.T))
        assert np.array_equal(ow.lm_head.q.view(np.int8), q) and np.array_equal(ow.lm_head.s, sc)
    prompt = np.random.default_rng(spec["seed"] % 1000).integers(0, cfg.vocab_size, spec["prompt"]).astype(np.int32)
    print(f"case {name}: oracle prefill of {spec['prompt']} tokens, and of two perturbed copies", flush=True)
    ref = OracleRun(cfg, ow, prompt)
    perturbed = [OracleRun(cfg, _perturbed(ow, seed), prompt) for seed in (1, 2)]
    return dict(name=name, spec=spec, cfg=cfg, dev=dev, prompt=prompt, ref=ref, perturbed=perturbed, ow=ow)


def _bound(model, ref_z, pert_z) -> float:
    spread = max(_rel(z, ref_z) for z in pert_z)
    return max(FLOOR, TOL_FACTOR * spread)


def _check_greedy(model, tokens):
    """tokens[0] from the prompt, tokens[i + 1] from decoding tokens[i]."""
    ref, pert = model["ref"], model["perturbed"]
    refs = [ref.logits] + ref.decode(tokens[:-1])
    perts = [[p.logits] + p.decode(tokens[:-1]) for p in pert]
    exact = 0
    for i, (tok, z) in enumerate(zip(tokens, refs)):
        best = int(np.argmax(z))
        if tok == best:
            exact += 1
            continue
        bound = _bound(model, z, [pz[i] for pz in perts])
        margin = float(z[best] - z[tok]) / float(np.abs(z).max())
        assert margin <= bound, (
            f"step {i}: GPU token {tok}, oracle argmax {best} (margin {margin:.3e} of max|logit| > {bound:.3e})")
    print(f"  greedy: {exact}/{len(tokens)} tokens are the oracle's argmax, the rest near-ties", flush=True)


def _run_engine(model, session):
    name = model["name"]
    prompt = model["prompt"]
    ref, pert = model["ref"], model["perturbed"]
    z = session.prefill(prompt)
    _close(z, ref.logits, _bound(model, ref.logits, [p.logits for p in pert]), f"{name} prompt logits")
    assert int(np.argmax(z)) == int(np.argmax(ref.logits))
    toks = [int(np.argmax(z))]
    pos = len(prompt)
    for i in range(LOGIT_STEPS):
        zi = session.forward_step(toks[-1], pos + i)
        zr = ref.decode(toks)[-1]
        bound = _bound(model, zr, [p.decode(toks)[-1] for p in pert])
        _close(zi, zr, bound, f"{name} decode step {i} logits")
        toks.append(int(np.argmax(zi)))
    gen, _ = session.generate(prompt, STEPS)
    gen = [int(t) for t in gen]
    assert gen[: len(toks)] == toks
    _check_greedy(model, gen)


@pytest.mark.timeout(900)
def test_resident_decoder_full_size(llama_module, model):
    spec = model["spec"]
    print(f"case {model['name']}: resident decoder", flush=True)
    s = llama_module.Session(model["dev"], llama_module.ENGINE_RESIDENT, spec["quant"], spec["block"],
                             max_seq=spec["prompt"] + STEPS + 8)
    try:
        _run_engine(model, s)
    finally:
        s.close()


@pytest.mark.timeout(900)
def test_graph_engine_full_size(llama_module, model):
    spec = model["spec"]
    print(f"case {model['name']}: graph engine", flush=True)
    s = llama_module.Session(model["dev"], llama_module.ENGINE_GRAPH, spec["quant"], spec["block"], False)
    try:
        _run_engine(model, s)
    finally:
        s.close()


@pytest.mark.timeout(900)
def test_resident_decoder_late_positions(llama_module, model):
    """The bench's last decode positions (TinyLlama 760..767 of max_seq 769,
    SmolLM2 248..255 of 257): teacher-forced steps against the oracle, and
    the HIP-graph generation of the same tokens."""
    import dataclasses

    spec, cfg, name = model["spec"], model["cfg"], model["name"]
    end = spec["prompt"] + spec["decode"]
    n = end - LATE_STEPS
    prompt = np.random.default_rng(spec["seed"] % 997).integers(0, cfg.vocab_size, n).astype(np.int32)
    print(f"case {name}: late positions {n}..{end - 1}, oracle prefill of {n} tokens (and two perturbed)", flush=True)
    ow = model["ow"]
    ref = OracleRun(cfg, ow, prompt)
    pert = [OracleRun(cfg, _perturbed(ow, seed), prompt) for seed in (3, 4)]
    s = llama_module.Session(model["dev"], llama_module.ENGINE_RESIDENT, spec["quant"], spec["block"], max_seq=end + 1)
    try:
        z = s.prefill(prompt)
        _close(z, ref.logits, _bound(model, ref.logits, [p.logits for p in pert]), f"{name} prompt of {n}")
        toks = [int(np.argmax(z))]
        for i in range(LATE_STEPS):
            zi = s.forward_step(toks[-1], n + i)
            zr = ref.decode(toks)[-1]
            _close(zi, zr, _bound(model, zr, [p.decode(toks)[-1] for p in pert]), f"{name} decode at {n + i}")
            toks.append(int(np.argmax(zi)))
        gen, _ = s.generate(prompt, LATE_STEPS - 1)
        assert [int(t) for t in gen] == toks[:LATE_STEPS]
    finally:
        s.close()


@pytest.mark.timeout(900)
def test_prompt_logits_meet_the_reference_criteria_exactly(llama_module, model):
    """Prompt logits of the resident decoder against the oracle run with the
    reference CPU QuantizedMatMul's own arithmetic (LINEAR_EXACT: exact
    codes and scales, no fp16 staging) under the reference's end-to-end
    criteria."""
    import dataclasses

    spec, cfg, name = model["spec"], model["cfg"], model["name"]
    ow = model["ow"]
    exact = lambda lin: dataclasses.replace(lin, mode=L.LINEAR_EXACT, _dense=None)  # noqa: E731
    ex = L.LlamaWeights(embed=ow.embed, final_norm=ow.final_norm, lm_head=exact(ow.lm_head), attn_norm=ow.attn_norm,
                        ffn_norm=ow.ffn_norm, wq=[exact(x) for x in ow.wq], wk=[exact(x) for x in ow.wk],
                        wv=[exact(x) for x in ow.wv], wo=[exact(x) for x in ow.wo], gate=[exact(x) for x in ow.gate],
                        up=[exact(x) for x in ow.up], down=[exact(x) for x in ow.down])
    print(f"case {name}: oracle prefill with the reference's QuantizedMatMul arithmetic", flush=True)
    ref, _ = L.prefill(cfg, ex, model["prompt"], last_only=True)
    ref = ref[0]
    s = llama_module.Session(model["dev"], llama_module.ENGINE_RESIDENT, spec["quant"], spec["block"],
                             max_seq=spec["prompt"] + 8)
    try:
        z = s.prefill(model["prompt"])
    finally:
        s.close()
    max_diff, rmse, _, cos = Q.metrics(ref, z)
    print(f"  {name}: cosine {cos:.6f}, rmse {rmse:.3e}, max diff {max_diff:.3e}, "
          f"max|logit| {float(np.abs(ref).max()):.3e}", flush=True)
    assert cos > 0.999
    assert rmse < 0.15
    assert int(np.argmax(z)) == int(np.argmax(ref))


@pytest.fixture(scope="module")
def llama_module(hip):
    from velomind_hip import llama as VL

    return VL
