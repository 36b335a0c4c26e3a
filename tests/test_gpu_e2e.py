"""End-to-end parity: random-init SmolLM2-135M-shape BitNet, greedy decode of 128
tokens from a 32-token random prompt.  The same model runs twice: every quantised BitLinear group
(RMSNorm/SubLN -> per-token int8 -> ternary linear -> rescale, and the MLP middle act(gate) * up ->
SubLN -> int8 -> down) once on libwfbitnet (separate or fused launches) and once on the CPU oracle;
the float glue (embedding, RoPE, attention, residuals, tied LM head) is the same code on the same
device in both runs.  Token ids and every per-layer int32 accumulator must be equal.
"""

import numpy as np
import pytest
import torch

from oracle.model_backend import OracleBackend as _OracleBackend

pytestmark = pytest.mark.gpu


def OracleBackend(model, dev):
    """The numpy-oracle backend over every ternary linear of the model (oracle/model_backend.py)."""
    return _OracleBackend(model.backend_linears, dev)


@pytest.mark.parametrize("fused", [False, True])
def test_greedy_decode_tokens_and_accumulators_match_oracle(pkg, dev, fused):
    M = pkg.model
    model = M.BitNetDecoder(M.SMOLLM2_135M, seed=0, device=dev)
    model.backend_linears = list(M.quantised_linears(model).values())
    prompt = torch.randint(0, M.SMOLLM2_135M.vocab_size, (1, 32), generator=torch.Generator().manual_seed(1))

    hip = M.HipBackend(out_dtype=torch.float32, keep_acc=True, fused=fused)
    model.backend = hip
    toks_hip = model.generate(prompt, 128).cpu()

    ref = OracleBackend(model, dev)
    model.backend = ref
    toks_ref = model.generate(prompt, 128).cpu()

    assert toks_hip.shape == (1, 128)
    assert torch.equal(toks_hip, toks_ref), f"first divergence at {int((toks_hip != toks_ref).nonzero()[0, 1])}"
    assert len(hip.acc_log) == len(ref.acc_log) == 128 * 30 * 7
    for i, (a, b) in enumerate(zip(hip.acc_log, ref.acc_log)):
        assert np.array_equal(a.cpu().numpy().astype(np.int64), b), f"accumulator mismatch at call {i}"
    # the generated text is not degenerate (random weights still give varied tokens)
    assert len(set(toks_hip[0].tolist())) > 4


def test_relu2_model_fused_matches_oracle(pkg, dev):
    """The relu(gate)^2 * up MLP of the BitNet b1.58 2B form (bitnet_fused_layer.cpp:200-204), small
    model, fused launches, prefill of 8 tokens as a batch of 2 plus 24 decode steps."""
    M = pkg.model
    cfg = M.BitNetConfig(vocab_size=2048, hidden_size=256, intermediate_size=640, num_layers=3, num_heads=4,
                         num_kv_heads=2, head_dim=64, rope_theta=10000.0, hidden_act="relu2")
    model = M.BitNetDecoder(cfg, seed=3, device=dev)
    model.backend_linears = list(M.quantised_linears(model).values())
    prompt = torch.randint(0, cfg.vocab_size, (2, 8), generator=torch.Generator().manual_seed(4))
    hip = M.HipBackend(out_dtype=torch.float32, keep_acc=True, fused=True)
    model.backend = hip
    toks_hip = model.generate(prompt, 24).cpu()
    ref = OracleBackend(model, dev)
    model.backend = ref
    toks_ref = model.generate(prompt, 24).cpu()
    assert torch.equal(toks_hip, toks_ref)
    assert len(hip.acc_log) == len(ref.acc_log)
    for a, b in zip(hip.acc_log, ref.acc_log):
        assert np.array_equal(a.cpu().numpy().astype(np.int64), b)


def test_ternary_lm_head_model_matches_oracle(pkg, dev):
    """An untied ternary LM head (the configs[4] form): greedy tokens from the fused linear+argmax kernel
    equal the oracle's argmax over exact logits, batch 3, 20 decode steps; every accumulator equal."""
    M = pkg.model
    cfg = M.BitNetConfig(vocab_size=3000, hidden_size=256, intermediate_size=512, num_layers=2, num_heads=4,
                         num_kv_heads=1, head_dim=64, rope_theta=500000.0, tie_embeddings=False, ternary_lm_head=True)
    model = M.BitNetDecoder(cfg, seed=9, device=dev)
    model.backend_linears = list(M.quantised_linears(model).values())
    prompt = torch.randint(0, cfg.vocab_size, (3, 6), generator=torch.Generator().manual_seed(10))
    hip = M.HipBackend(out_dtype=torch.float32, keep_acc=True, fused=True)
    model.backend = hip
    toks_hip = model.generate(prompt, 20).cpu()
    ref = OracleBackend(model, dev)
    model.backend = ref
    toks_ref = model.generate(prompt, 20).cpu()
    assert torch.equal(toks_hip, toks_ref)
    assert len(hip.acc_log) == len(ref.acc_log)
    for a, b in zip(hip.acc_log, ref.acc_log):
        assert np.array_equal(a.cpu().numpy().astype(np.int64), b)
    assert len(set(toks_hip.flatten().tolist())) > 4


def test_decode_graph_replays_match_eager(pkg, dev):
    """The decode step captured once in a HIP graph and replayed gives the same tokens as running it
    directly; two graph runs with eager work between them (each replay's token is checked)."""
    M = pkg.model
    cfg = M.BitNetConfig(vocab_size=4096, hidden_size=576, intermediate_size=1536, num_layers=4, num_heads=9,
                         num_kv_heads=3, head_dim=64, rope_theta=100000.0)
    model = M.BitNetDecoder(cfg, seed=2, device=dev, backend=M.HipBackend(out_dtype=torch.float32, fused=True))
    prompt = torch.randint(0, cfg.vocab_size, (2, 16), generator=torch.Generator().manual_seed(3))
    eager = model.generate(prompt, 40).cpu()
    g1 = model.generate(prompt, 40, graph=True).cpu()
    torch.cuda.synchronize()
    eager2 = model.generate(prompt[:, :9], 12).cpu()  # other eager work in between
    g2 = model.generate(prompt, 40, graph=True).cpu()
    assert torch.equal(eager, g1), f"graph run 1 diverges at step {int((eager != g1).nonzero()[0, 1])}"
    assert torch.equal(eager, g2)
    assert eager2.shape == (2, 12)
    assert len(set(eager[0].tolist())) > 3


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_hip_decode_attention_matches_torch_decode(pkg, dev, dtype):
    """The decode step with the fused rotary + cache-append + GQA attention kernel against the same
    step as torch ops, teacher-forced on the same ids for 12 steps after a shared prefill: the caches
    the two paths append agree exactly (same rotary arithmetic) and the logits agree to a tolerance
    (attention is float math in a different order; an activation code can move by one at a
    rounding boundary)."""
    M = pkg.model
    cfg = M.BitNetConfig(vocab_size=4096, hidden_size=512, intermediate_size=1024, num_layers=3, num_heads=8,
                         num_kv_heads=2, head_dim=128, rope_theta=500000.0)
    runs = {}
    prompt = torch.randint(0, cfg.vocab_size, (3, 20), generator=torch.Generator().manual_seed(6)).to(dev)
    feed = torch.randint(0, cfg.vocab_size, (3, 12), generator=torch.Generator().manual_seed(7)).to(dev)
    for mode in ("torch", "hip"):
        model = M.BitNetDecoder(cfg, seed=5, device=dev, dtype=dtype, decode_attention=mode,
                                backend=M.HipBackend(out_dtype=dtype, fused=True))
        with torch.no_grad():
            model.reset(3, 32)
            logits = [model.forward(prompt, 0)]
            pos = torch.full((3,), 20, dtype=torch.long, device=dev)
            for s in range(12):
                logits.append(model.decode_step(feed[:, s:s + 1], pos))
                pos += 1
        runs[mode] = (torch.stack(logits).cpu(), [c.cpu() for kv in model.kv for c in kv])
    lt, ct = runs["torch"]
    lh, ch = runs["hip"]
    assert torch.equal(lt[0], lh[0])  # prefill is the same torch code
    for a, b in zip(ct, ch):
        assert torch.equal(a[:, :, :20], b[:, :, :20])
    # first decode step: identical inputs, so the appended layer-0 key/value rows are bit-identical
    assert torch.equal(ct[0][:, :, 20], ch[0][:, :, 20]) and torch.equal(ct[1][:, :, 20], ch[1][:, :, 20])
    span = float(lt.abs().max())
    diff = (lt - lh).abs()
    # a misplaced head, position or key would move logits by O(span); rounding-boundary code flips in
    # the int8 activations downstream move them by well under 1%
    assert float(diff.max()) <= (2e-2 if dtype == torch.float32 else 5e-2) * span
    assert float(diff.mean()) <= (2e-3 if dtype == torch.float32 else 1e-2) * span


def test_hip_prefill_attention_matches_torch_prefill(pkg, dev):
    """A bf16 model's prompt forward with the matrix-core prefill attention kernel against the same
    forward as torch ops: layer 0's cache is bit-identical (same inputs, same rotary arithmetic; deeper
    layers see hidden states that already differ by float rounding) and the logits agree to the float
    tolerance of the decode comparison; greedy decode then continues from either cache."""
    M = pkg.model
    cfg = M.BitNetConfig(vocab_size=4096, hidden_size=512, intermediate_size=1024, num_layers=3, num_heads=8,
                         num_kv_heads=2, head_dim=128, rope_theta=500000.0)
    prompt = torch.randint(0, cfg.vocab_size, (3, 45), generator=torch.Generator().manual_seed(9)).to(dev)
    runs = {}
    for mode in ("torch", "hip"):
        model = M.BitNetDecoder(cfg, seed=5, device=dev, dtype=torch.bfloat16, prefill_attention=mode,
                                backend=M.HipBackend(out_dtype=torch.bfloat16, fused=True))
        assert model._hip_prefill() == (mode == "hip")
        with torch.no_grad():
            model.reset(3, 64)
            logits = model.forward(prompt, 0)
            toks = model.generate(prompt, 6)
        runs[mode] = (logits.cpu(), [c.cpu() for kv in model.kv for c in kv], toks.cpu())
    lt, ct, tt = runs["torch"]
    lh, ch, th = runs["hip"]
    assert torch.equal(ct[0][:, :, :45], ch[0][:, :, :45]) and torch.equal(ct[1][:, :, :45], ch[1][:, :, :45])
    for a, b in zip(ct[2:], ch[2:]):
        assert float((a.float() - b.float()).abs().max()) <= 5e-2 * float(a.float().abs().max())
    span = float(lt.abs().max())
    diff = (lt - lh).abs()
    assert float(diff.max()) <= 5e-2 * span
    assert float(diff.mean()) <= 1e-2 * span
    assert tt.shape == th.shape == (3, 6)


def test_host_copy_runs_the_same_model(pkg, dev):
    """on_host (the end-to-end CPU baseline): the same weights with torch-CPU float glue and the oracle
    BitLinears give the GPU model's prefill logits to a float tolerance, and decode on the host."""
    M = pkg.model
    cfg = M.BitNetConfig(vocab_size=2048, hidden_size=256, intermediate_size=512, num_layers=2, num_heads=4,
                         num_kv_heads=2, head_dim=64, rope_theta=10000.0)
    model = M.BitNetDecoder(cfg, seed=8, device=dev, backend=M.HipBackend(out_dtype=torch.float32, fused=True))
    lins = list(M.quantised_linears(model).values())
    host = model.on_host(_OracleBackend(lins, "cpu"))
    prompt = torch.randint(0, cfg.vocab_size, (2, 10), generator=torch.Generator().manual_seed(2))
    with torch.no_grad():
        model.reset(2, 16)
        lg = model.forward(prompt.to(dev), 0).cpu()
        host.reset(2, 16)
        lh = host.forward(prompt, 0)
    assert lh.device.type == "cpu"
    assert float((lg - lh).abs().max()) <= 2e-2 * float(lg.abs().max())
    toks = host.generate(prompt, 5)
    assert toks.shape == (2, 5) and toks.device.type == "cpu"


def _ref_golden():
    from pathlib import Path

    return np.load(Path(__file__).resolve().parent / "golden" / "ref_e2e_smollm2.npz", allow_pickle=False)


def _model_from_ref_state(pkg, dev, g):
    M = pkg.model
    cfg = M.SMOLLM2_135M
    return M.BitNetDecoder.from_float_state(M.random_float_state(cfg, int(g["seed"][0])), cfg, device=dev,
                                            backend=M.HipBackend(out_dtype=torch.float32, fused=True))


def test_layers_match_reference_stage1_model(pkg, dev):
    """configs[0] against the reference's OWN model, layer by layer: tests/golden/ref_e2e_smollm2.npz holds
    the residual stream entering and leaving layers 0, 1, 10, 15, 20, 29 of transformers' LlamaForCausalLM
    converted by the reference's convert_model_to_bitnet (stage1.py:169-214; reference BitLinear and SubLN
    forwards, fp32, eager attention) on the 32-token prompt, written in the build container by
    tests/golden/make_e2e_golden.py from the float weights random_float_state(seed).  The HIP model built
    from the same floats (absmean-ternarised and packed on the device) maps each layer's input to its
    output within 1e-2 normwise, and at least half the layers within 1e-6: the two float paths round
    differently (dequantised fp32 F.linear there, exact integer accumulators here), which moves an int8
    activation code across a rounding boundary only now and then (layers 0, 10 and 29 flip a few).  A wrong RoPE theta (1e4) or SubLN eps
    (1e-5) gives 4.5e-3 / 9e-4 on layer 15 where this path gives about 1e-7 (measured on the CPU with the
    oracle backend and the same float code)."""
    g = _ref_golden()
    model = _model_from_ref_state(pkg, dev, g)
    errs = []
    with torch.no_grad():
        for li in g["layers"].tolist():
            x_in = torch.from_numpy(g[f"layer{li}_in"])[None]
            want = torch.from_numpy(g[f"layer{li}_out"]).double()
            model.reset(1, x_in.shape[1])
            got = model.forward_layers(x_in, 0, li, li + 1)[0].cpu().double()
            errs.append(float((got - want).norm() / want.norm()))
    print("per-layer normwise differences:", dict(zip(g["layers"].tolist(), [f"{e:.1e}" for e in errs])), flush=True)
    assert max(errs) <= 1e-2, errs
    assert sorted(errs)[len(errs) // 2 - 1] <= 1e-6, errs  # half the layers flip no code: fp32 rounding only


def test_logits_match_reference_stage1_model_within_its_own_noise(pkg, dev):
    """configs[0] end to end against the reference's OWN model (see the test above): prompt logits and
    teacher-forced logits (at the reference's top-5 ids of each of its 128 greedy steps, fed its tokens)
    differ from the reference's by no more than twice what the reference moves by itself when its input
    embeddings get rounding-level noise (x (1 + 1e-7 N(0,1)), recorded in the fixture: 0.14 / 0.11 on
    logits of range 2.0).  Code flips at rounding boundaries compound over 30 layers, so identical free-
    running tokens are not a property of this random-init model: under that noise the reference's own
    first greedy token already changes.  Where the reference's top-2 gap at a step exceeds twice its own
    noise, the greedy pick must be the reference's."""
    g = _ref_golden()
    model = _model_from_ref_state(pkg, dev, g)
    prompt = torch.from_numpy(g["prompt"])[None]
    ref_toks = g["tokens"]
    noise_prefill = float(np.abs(g["perturbed_prefill_logits"] - g["prefill_logits"]).max())
    noise_tf = float(np.abs(g["perturbed_top5_logits"] - g["top5_logits"]).max())
    with torch.no_grad():
        model.reset(1, prompt.shape[1] + len(ref_toks))
        logits = model.forward(prompt.to(dev), 0)
        d_prefill = float(np.abs(logits[0].cpu().numpy() - g["prefill_logits"]).max())
        pos = torch.full((1,), prompt.shape[1], dtype=torch.long, device=dev)
        worst, robust = 0.0, 0
        for t in range(len(ref_toks)):
            row = logits[0].cpu().numpy()
            worst = max(worst, float(np.abs(row[g["top5_ids"][t]] - g["top5_logits"][t]).max()))
            gap = float(g["top5_logits"][t, 0] - g["top5_logits"][t, 1])
            if gap > 2 * noise_tf:
                robust += 1
                assert int(row.argmax()) == int(ref_toks[t]), f"step {t}: greedy pick differs where the gap is {gap:.3f}"
            if t + 1 < len(ref_toks):
                logits = model.decode_step(torch.tensor([[int(ref_toks[t])]], device=dev), pos)
                pos += 1
    print(f"prompt logits: {d_prefill:.3e} (reference self-noise {noise_prefill:.3e}); teacher-forced top-5: "
          f"{worst:.3e} (self-noise {noise_tf:.3e}); {robust} robust steps", flush=True)
    assert d_prefill <= 2 * noise_prefill
    assert worst <= 2 * noise_tf
