"""The native engine (include/wfbitnet_engine.h, the reference's engine C ABI) on the GPU.

Its greedy tokens must equal, id for id, those of the Python model with the fused HIP backend and bf16
glue on the same SGLBITNT weights (model.py: BitNetDecoder.generate with the same KV cache length), itself
pinned to the CPU oracle by test_gpu_e2e.py.  The engine issues the same libwfbitnet calls per layer, so
this checks its loading (segment concatenation, bf16 conversion, rotary tables), its batched prompt pass,
its graph-replayed decode steps and its greedy / EOS / decode_step bookkeeping against the reference's
semantics (SGB/sgl-kernel/csrc/inference/bitnet_engine.cpp:742-893).
"""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _model(M, dev, cfg, seed, dense_head=False):
    be = M.HipBackend(out_dtype=torch.bfloat16, fused=True)
    if dense_head:
        st = M.random_float_state(cfg, seed)
        return M.BitNetDecoder.from_float_state(st, cfg, device=dev, dtype=torch.bfloat16, backend=be)
    return M.BitNetDecoder(cfg, seed=seed, device=dev, dtype=torch.bfloat16, backend=be)


def _prompt(cfg, n, seed):
    return torch.randint(0, cfg.vocab_size, (1, n), generator=torch.Generator().manual_seed(seed))


SMALL = dict(vocab_size=2048, hidden_size=256, intermediate_size=640, num_layers=3, num_heads=4, num_kv_heads=2,
             head_dim=64, rope_theta=10000.0)


def _cases(M):
    return {
        # SmolLM2-135M shape, tied bf16 head, SwiGLU
        "smollm2": (M.SMOLLM2_135M, False),
        # BitNet b1.58 2B form (relu^2) with an untied ternary head
        "relu2_ternary_head": (M.BitNetConfig(**SMALL, hidden_act="relu2", tie_embeddings=False,
                                              ternary_lm_head=True), False),
        # untied dense float head
        "dense_head": (M.BitNetConfig(**dict(SMALL, num_kv_heads=4), tie_embeddings=False), True),
        # FFN width not a multiple of 32: the gate|up outputs and the gated row quantiser at every M
        "ffn_648": (M.BitNetConfig(**dict(SMALL, intermediate_size=648)), False),
    }


# the small models at every prompt path, the SmolLM2 shape at one
_GREEDY_CASES = [("smollm2", 40)] + [(c, p) for c in ("relu2_ternary_head", "dense_head", "ffn_648") for p in (5, 40, 100)]


@pytest.mark.parametrize("case,plen", _GREEDY_CASES)
def test_engine_greedy_tokens_equal_the_model(pkg, dev, tmp_path, case, plen):
    """Prompt lengths 5 / 40 / 100 take the three prompt paths (norm fused into the linear for <= 16 rows,
    the gated gate|up epilogue for <= 64, the prefill GEMMs beyond); 70 decode steps cross two 32-step
    chunks."""
    M = pkg.model
    cfg, dense = _cases(M)[case]
    model = _model(M, dev, cfg, seed=11, dense_head=dense)
    path = tmp_path / "m.bin"
    model.save_sglbitnt(path)
    max_len, new = 192, 70
    prompt = _prompt(cfg, plen, 3)
    want = model.generate(prompt, new, max_len=max_len)[0].tolist()
    with pkg.NativeEngine(str(path), max_seq_len=max_len) as eng:
        assert (eng.vocab_size, eng.hidden_size, eng.num_layers, eng.max_seq_len, eng.num_kv_heads) == (
            cfg.vocab_size, cfg.hidden_size, cfg.num_layers, max_len, cfg.num_kv_heads)
        got = eng.generate(prompt[0].tolist(), max_tokens=new)
        assert got == want, f"first divergence at {next(i for i, (a, b) in enumerate(zip(got, want)) if a != b)}"
        # a second generation on the same engine starts from a reset cache
        assert eng.generate(prompt[0].tolist(), max_tokens=new) == want
        assert len(set(got)) > 4


def test_engine_llama3_width_matches_the_model(pkg, dev, tmp_path):
    """Llama-3-8B layer widths (hidden 4096, 32/8 heads of 128, FFN 14336) at 2 layers with a ternary head over
    40000 rows (the persistent head kernel): the fused norm before q|k|v, o and gate|up, the two-call path
    before down (K 14336)."""
    M = pkg.model
    cfg = M.BitNetConfig(vocab_size=40000, hidden_size=4096, intermediate_size=14336, num_layers=2, num_heads=32,
                         num_kv_heads=8, head_dim=128, rope_theta=500000.0, tie_embeddings=False,
                         ternary_lm_head=True)
    model = M.BitNetDecoder(cfg, seed=5, device=dev, dtype=torch.bfloat16, init_on_device=True,
                            backend=M.HipBackend(out_dtype=torch.bfloat16, fused=True))
    path = tmp_path / "llama.bin"
    model.save_sglbitnt(path)
    prompt = _prompt(cfg, 80, 9)
    want = model.generate(prompt, 40, max_len=256)[0].tolist()
    with pkg.NativeEngine(str(path), max_seq_len=256) as eng:
        assert eng.generate(prompt[0].tolist(), max_tokens=40) == want


def test_engine_bitnet_2b_full_size_matches_the_model(pkg, dev, tmp_path):
    """The BitNet b1.58 2B4T shape at full size (30 layers, relu^2, GQA 20/5, 128256-row tied bf16 head): 64-token
    prompt, 16 tokens -- the first row of the published A100 latency table -- equal to the Python model's."""
    M = pkg.model
    cfg = M.BITNET_2B
    model = M.BitNetDecoder(cfg, seed=4, device=dev, dtype=torch.bfloat16, init_on_device=True,
                            backend=M.HipBackend(out_dtype=torch.bfloat16, fused=True))
    path = tmp_path / "bitnet2b.bin"
    model.save_sglbitnt(path)
    prompt = _prompt(cfg, 64, 12)
    want = model.generate(prompt, 16, max_len=128)[0].tolist()
    del model
    torch.cuda.empty_cache()
    with pkg.NativeEngine(str(path), max_seq_len=128) as eng:
        assert eng.generate(prompt[0].tolist(), max_tokens=16) == want


def test_prefill_and_decode_steps_equal_generate(pkg, dev, tmp_path):
    """bitnet_prefill then bitnet_decode_step(position = prompt + i): the reference's step contract (pick from
    the logits of the last token run, run the pick at `position`) gives generate's tokens."""
    M = pkg.model
    cfg = M.BitNetConfig(**SMALL, hidden_act="relu2")
    model = _model(M, dev, cfg, seed=2)
    path = tmp_path / "m.bin"
    model.save_sglbitnt(path)
    prompt = _prompt(cfg, 12, 4)[0].tolist()
    with pkg.NativeEngine(str(path), max_seq_len=96) as eng:
        want = eng.generate(prompt, max_tokens=20)
        eng.prefill(prompt)
        got = [eng.decode_step(len(prompt) + i) for i in range(20)]
        assert got == want
        # generate, then steps continue where it stopped (its last token was also run)
        eng.generate(prompt, max_tokens=10)
        assert [eng.decode_step(len(prompt) + 10 + i) for i in range(10)] == want[10:20]


def test_eos_stops_generation_and_keeps_the_reference_state(pkg, dev, tmp_path):
    """With eos_token_id set, generate returns the tokens up to and including the first EOS and stops before
    running it (bitnet_engine.cpp:791-795): the next decode_step picks the EOS again from the same logits,
    the one after continues the unrestricted sequence.  EOS as the first token (the prompt's state) and inside
    the second 32-token chunk (a hidden state restored from the ring)."""
    M = pkg.model
    cfg = M.BitNetConfig(**SMALL)
    model = _model(M, dev, cfg, seed=7)
    free_path = tmp_path / "free.bin"
    model.save_sglbitnt(free_path)
    prompt = _prompt(cfg, 9, 5)[0].tolist()
    n = len(prompt)
    with pkg.NativeEngine(str(free_path), max_seq_len=160) as eng:
        full = eng.generate(prompt, max_tokens=100)
    picks = [0] + [i for i in range(33, 64) if full[i] not in full[:i]][:1]
    assert len(picks) == 2, "no fresh token inside the second chunk to use as EOS"
    for e in picks:
        path = tmp_path / f"eos{e}.bin"
        model.save_sglbitnt(path, config_overrides={"eos_token_id": [full[e], 2 ** 30]})
        with pkg.NativeEngine(str(path), max_seq_len=160) as eng:
            got = eng.generate(prompt, max_tokens=100)
            assert got == full[:e + 1]
            assert eng.decode_step(n + e) == full[e]
            assert [eng.decode_step(n + e + 1 + i) for i in range(5)] == full[e + 1:e + 6]


def test_sampling_is_seeded_and_nucleus_of_one_is_greedy(pkg, dev, tmp_path):
    """temperature > 0: the engine's mt19937(42) makes a fresh engine repeat its samples; a nucleus smaller
    than the top probability reproduces greedy decoding (fp32 logits of the tied head, no ties)."""
    M = pkg.model
    cfg = M.BitNetConfig(**SMALL)
    model = _model(M, dev, cfg, seed=8)
    path = tmp_path / "m.bin"
    model.save_sglbitnt(path)
    prompt = _prompt(cfg, 10, 6)[0].tolist()
    runs = []
    for _ in range(2):
        with pkg.NativeEngine(str(path), max_seq_len=64) as eng:
            runs.append(eng.generate(prompt, temperature=0.8, top_p=0.95, max_tokens=24))
            greedy = eng.generate(prompt, max_tokens=24)
            narrow = eng.generate(prompt, temperature=1.0, top_p=1e-9, max_tokens=24)
            assert narrow == greedy
    assert runs[0] == runs[1] and len(runs[0]) == 24
    assert all(0 <= t < cfg.vocab_size for t in runs[0])
    assert runs[0] != greedy  # sampling at 0.8 departs from greedy somewhere in 24 steps


def test_engine_errors_on_the_device(pkg, dev, tmp_path):
    M = pkg.model
    cfg = M.BitNetConfig(**SMALL)
    model = _model(M, dev, cfg, seed=1)
    path = tmp_path / "m.bin"
    model.save_sglbitnt(path)
    with pkg.NativeEngine(str(path), max_seq_len=32) as eng:
        with pytest.raises(RuntimeError, match="no prompt has been run"):
            eng.decode_step(0)
        with pytest.raises(RuntimeError, match="exceeds max_seq_len"):
            eng.generate([1, 2, 3], max_tokens=30)
        with pytest.raises(RuntimeError, match="out of range"):
            eng.generate([1, cfg.vocab_size], max_tokens=2)
        with pytest.raises(RuntimeError, match="num_input_tokens must be >= 1"):
            eng.generate([], max_tokens=2)
        eng.prefill([1, 2, 3])
        with pytest.raises(RuntimeError, match="outside"):
            eng.decode_step(32)
        eng.reset()
        with pytest.raises(RuntimeError, match="no prompt has been run"):
            eng.decode_step(3)
        assert eng.generate([4, 5], max_tokens=0) == []


@pytest.mark.parametrize("after", [0, 3, 7])
def test_failed_prompt_buffer_growth_leaves_no_state(pkg, dev, tmp_path, after):
    """A prompt longer than every earlier one grows the prompt buffers (7 device buffers, then the pinned id
    buffer).  When one of those allocations fails (the first, a middle one, the pinned one) the call returns -1
    with the allocator's message and keeps no buffers, so later prompts, shorter or longer, allocate again and
    give a fresh engine's tokens."""
    M = pkg.model
    cfg = M.BitNetConfig(**SMALL, hidden_act="relu2")
    model = _model(M, dev, cfg, seed=2)
    path = tmp_path / "m.bin"
    model.save_sglbitnt(path)
    short = _prompt(cfg, 6, 4)[0].tolist()
    longp = _prompt(cfg, 50, 5)[0].tolist()
    with pkg.NativeEngine(str(path), max_seq_len=96) as ref:
        want_long = ref.generate(longp, max_tokens=12)
    with pkg.NativeEngine(str(path), max_seq_len=96) as ref:
        want_short = ref.generate(short, max_tokens=12)
    with pkg.NativeEngine(str(path), max_seq_len=96) as eng:
        assert eng.generate(short, max_tokens=12) == want_short
        pkg.engine.fail_alloc_after(after)
        try:
            with pytest.raises(RuntimeError, match="allocation failure injected"):
                eng.generate(longp, max_tokens=12)
        finally:
            pkg.engine.fail_alloc_after(-1)
        with pytest.raises(RuntimeError, match="no prompt has been run"):
            eng.decode_step(len(longp))
        assert eng.generate(short, max_tokens=12) == want_short
        assert eng.generate(longp, max_tokens=12) == want_long


def test_engine_calls_keep_the_callers_device(pkg, dev, tmp_path):
    """Every engine entry point runs on the engine's device and leaves the calling thread's current device as
    it found it (with one GPU: the same device before and after each call, also after a failed call)."""
    M = pkg.model
    cfg = M.BitNetConfig(**SMALL)
    model = _model(M, dev, cfg, seed=1)
    path = tmp_path / "m.bin"
    model.save_sglbitnt(path)
    before = torch.cuda.current_device()
    with pkg.NativeEngine(str(path), max_seq_len=32) as eng:
        eng.generate([1, 2, 3], max_tokens=4)
        assert torch.cuda.current_device() == before
        with pytest.raises(RuntimeError):
            eng.decode_step(40)
        assert torch.cuda.current_device() == before
    assert torch.cuda.current_device() == before


@pytest.mark.parametrize("case,plen", [("smollm2", 40), ("relu2_ternary_head", 5), ("relu2_ternary_head", 100),
                                       ("dense_head", 40)])
def test_engine_fp32_glue_matches_the_fp32_model(pkg, dev, tmp_path, case, plen):
    """A file whose config says torch_dtype float32 runs the engine's float glue in fp32 -- embedding, norms,
    residual stream, KV cache, attention and a dense head, as the reference engine computes
    (bitnet_engine.cpp:107, 146-150, 289, 490-554) -- with the prompt's attention as one decode attention per
    position.  Its greedy tokens equal the fp32 Python model's (HipBackend fp32, fused, prompt attention by
    steps), id for id; the same weights in a bf16 file give the bf16 model's tokens."""
    M = pkg.model
    cfg, dense = _cases(M)[case]
    be = M.HipBackend(out_dtype=torch.float32, fused=True)
    if dense:
        model = M.BitNetDecoder.from_float_state(M.random_float_state(cfg, 11), cfg, device=dev, dtype=torch.float32,
                                                 backend=be, prefill_attention="steps")
    else:
        model = M.BitNetDecoder(cfg, seed=11, device=dev, dtype=torch.float32, backend=be, prefill_attention="steps")
    path = tmp_path / "m32.bin"
    model.save_sglbitnt(path)
    max_len, new = 192, 40
    prompt = _prompt(cfg, plen, 3)
    want = model.generate(prompt, new, max_len=max_len)[0].tolist()
    with pkg.NativeEngine(str(path), max_seq_len=max_len) as eng:
        got = eng.generate(prompt[0].tolist(), max_tokens=new)
        assert got == want, f"first divergence at {next(i for i, (a, b) in enumerate(zip(got, want)) if a != b)}"
        eng.prefill(prompt[0].tolist())
        assert [eng.decode_step(plen + i) for i in range(8)] == want[:8]
    assert len(set(want)) > 4
