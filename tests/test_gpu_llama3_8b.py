"""the Llama-3-8B-architecture BitNet (hidden 4096, 32/8 heads, FFN 14336, vocab 128256, every
linear ternary) on the HIP path -- 8 prompts x 256 tokens of prefill (one M = 2048 GEMM per projection),
then batch-8 greedy decode.

(a) Full width at reduced depth (4 layers): token ids and every int32 accumulator of every quantised
    call (prefill and 8 decode steps, LM head included) equal the CPU oracle backend's
    (oracle/model_backend.py), with the same float glue on both sides.
(b) Full depth (32 layers): the production path (fused launches, bf16) gives the same tokens eagerly,
    from a HIP graph, and through the unfused launches; on the unfused run, sampled calls of every
    projection type are checked against the oracle at their real shapes -- the row-sum identity
    sum_n acc[m, n] = a[m] . colsum(W) over the whole output, 16 rows exactly, and the stored bf16
    outputs (and residual adds) against the closed-form rescale of the accumulators -- and the LM
    head's greedy token against the argmax of the oracle's exact logits.
Reference loop: SGB/sgl-kernel/csrc/inference/bitnet_engine.cpp:742-823.
"""

import dataclasses

import numpy as np
import pytest
import torch

from oracle import bitnet_oracle as orc
from oracle.model_backend import OracleBackend

pytestmark = pytest.mark.gpu

BATCH, PROMPT = 8, 256


def _prompt(vocab, seed=5):
    return torch.randint(0, vocab, (BATCH, PROMPT), generator=torch.Generator().manual_seed(seed))


def test_llama3_8b_width_four_layers_tokens_and_accumulators_match_oracle(pkg, dev):
    M = pkg.model
    cfg = dataclasses.replace(M.LLAMA3_8B, num_layers=4)
    model = M.BitNetDecoder(cfg, seed=0, device=dev, dtype=torch.bfloat16, init_on_device=True)
    lins = list(M.quantised_linears(model).values())
    prompt = _prompt(cfg.vocab_size)
    new = 9  # the prompt's token + 8 decode steps

    hip = M.HipBackend(out_dtype=torch.float32, keep_acc=True, fused=False)
    model.backend = hip
    toks_hip = model.generate(prompt, new).cpu()
    print(f"llama3-8b x4 layers: HIP done, {len(hip.acc_log)} accumulator tensors", flush=True)

    ref = OracleBackend(lins, dev)
    model.backend = ref
    toks_ref = model.generate(prompt, new).cpu()
    print("llama3-8b x4 layers: oracle done", flush=True)

    assert toks_hip.shape == (BATCH, new)
    assert torch.equal(toks_hip, toks_ref), f"tokens differ: {toks_hip.tolist()} vs {toks_ref.tolist()}"
    # per layer 7 projections, plus the LM head, for the prefill and each decode step
    assert len(hip.acc_log) == len(ref.acc_log) == new * (7 * cfg.num_layers + 1)
    for i, (a, b) in enumerate(zip(hip.acc_log, ref.acc_log)):
        assert np.array_equal(a.cpu().numpy().astype(np.int64), b), f"accumulator mismatch at call {i} {tuple(b.shape)}"
    assert len(set(toks_hip.flatten().tolist())) > 8


class _SampledChecks:
    """Mixin over HipBackend (unfused, bf16 outputs): for calls of the projections named in ``sample``
    (names of quantised_linears), recompute the accumulators of the same call and check them, and the
    outputs the model used."""

    def setup(self, pkg, names, rng):
        self.pkg, self.names, self.rng, self.sample, self.done = pkg, names, rng, set(), []
        self._w = {}

    def _unpacked(self, lin):
        w = self._w.get(id(lin))
        if w is None:
            w = orc.unpack_i2s(lin.qweight.cpu().numpy())
            self._w = {id(lin): w}  # keep one at a time (host memory)
        return w

    def _check(self, q, a_scale, lin, y, residual):
        name = self.names[id(lin)]
        _, acc = self.pkg.bitnet_linear(lin.qweight, q, lin.scale, a_scale=a_scale, out_dtype=torch.float32,
                                        return_acc=True)
        m, n = acc.shape
        w = self._unpacked(lin)
        colsum = w.astype(np.int64).sum(axis=0)
        qn = q.cpu().numpy()
        accn = acc.cpu().numpy().astype(np.int64)
        assert np.array_equal(accn.sum(axis=1), qn.astype(np.int64) @ colsum), f"{name} M={m}: row-sum identity"
        rows = np.unique(np.concatenate([[0, m - 1], self.rng.choice(m, min(m, 14), replace=False)]))
        want = (qn[rows].astype(np.float32) @ w.T.astype(np.float32)).astype(np.int64)
        assert np.array_equal(accn[rows], want), f"{name} M={m}: sampled rows differ from the oracle"
        # the output the model used: fp32 rescale (acc * w_scale) * a_scale, + residual in fp32, rounded
        y32 = acc.float() * lin.scale * a_scale[:, None]
        if residual is not None:
            y32 = y32 + residual.float()
        assert torch.equal(y, y32.to(y.dtype)), f"{name} M={m}: stored outputs differ from the rescale"
        self.done.append((name.split(".")[-1], m))

    def _linears(self, q, a_scale, linears):
        outs = super()._linears(q, a_scale, linears)
        for lin, y in zip(linears, outs):
            if self.names[id(lin)] in self.sample:
                self._check(q, a_scale, lin, y, None)
        return outs

    def _linear_residual(self, q, a_scale, linear, residual):
        out = super()._linear_residual(q, a_scale, linear, residual)
        if self.names[id(linear)] in self.sample:
            self._check(q, a_scale, linear, out, residual)
        return out

    def norm_linear_argmax(self, x, norm_weight, eps, linear):
        tok = super().norm_linear_argmax(x, norm_weight, eps, linear)
        if "lm_head" in self.sample:
            q, a_scale = self.pkg.rmsnorm_quantize_i8(x, norm_weight, eps=eps, k_pad=linear.k_pad)
            w = self._unpacked(linear).astype(np.float32)
            acc = (q.cpu().numpy().astype(np.float32) @ w.T).astype(np.int64)
            logits = orc.rescale(acc, np.float32(linear.scale.item()), a_scale.cpu().numpy())  # fp32, as compared
            assert np.array_equal(tok.cpu().numpy(), logits.argmax(axis=1)), "LM head token != oracle argmax"
            self.done.append(("lm_head", x.shape[0]))
        return tok


def test_llama3_8b_full_depth_prefill_and_decode(pkg, dev):
    M = pkg.model
    cfg = M.LLAMA3_8B
    model = M.BitNetDecoder(cfg, seed=0, device=dev, dtype=torch.bfloat16, init_on_device=True,
                            backend=M.HipBackend(out_dtype=torch.bfloat16, fused=True))
    prompt = _prompt(cfg.vocab_size).to(dev)
    new = 17  # 16 decode steps
    eager = model.generate(prompt, new).cpu()
    graph = model.generate(prompt, new, graph=True).cpu()
    print("llama3-8b full depth: fused eager / graph done", flush=True)
    assert torch.equal(eager, graph), "graph replays diverge from eager decoding"

    Sampled = type("Sampled", (_SampledChecks, M.HipBackend), {})
    be = Sampled(out_dtype=torch.bfloat16, fused=False)
    be.setup(pkg, {id(l): n for n, l in M.quantised_linears(model).items()}, np.random.default_rng(0))
    model.backend = be
    projs = ("q", "k", "v", "o", "gate", "up", "down")
    with torch.no_grad():
        model.reset(BATCH, PROMPT + new)
        # prefill: every projection of layers 0 and 31 (M = 2048) and the LM head
        be.sample = {f"layers.{li}.{p}" for li in (0, 31) for p in projs} | {"lm_head"}
        nxt = model.forward(prompt, 0, tokens=True)
        print(f"llama3-8b full depth: prefill checks {len(be.done)}", flush=True)
        toks = [nxt]
        ids = nxt[:, None].clone()
        pos = torch.full((BATCH,), PROMPT, dtype=torch.long, device=dev)
        for s in range(new - 1):
            # decode step 3: every projection of layer 16 (M = 8) and the LM head
            be.sample = ({f"layers.16.{p}" for p in projs} | {"lm_head"}) if s == 3 else set()
            nxt = model.decode_step(ids, pos, tokens=True)
            toks.append(nxt)
            ids = nxt[:, None].clone()
            pos += 1
    unfused = torch.stack(toks, dim=1).cpu()
    kinds = set(be.done)
    assert kinds == {(p, BATCH * PROMPT) for p in projs} | {(p, BATCH) for p in projs} | {("lm_head", BATCH)}, kinds
    assert len(be.done) == 2 * 7 + 1 + 7 + 1
    assert torch.equal(unfused, eager), "unfused launches give different tokens from the fused path"
    assert len(set(eager.flatten().tolist())) > 16


def test_llama3_8b_full_depth_2048_token_prompts(pkg, dev):
    """configs[4] at its other reading: 8 prompts of 2048 tokens each (16384 prompt tokens, one M = 16384 GEMM
    per projection), then decode steps over 2048+ keys per sequence.  Eager and graph-replayed decoding give
    the same tokens; on an unfused run every projection of layer 0 at M = 16384, every projection of layer 31
    at the second decode step (M = 8) and the LM head are checked against the oracle as above."""
    M = pkg.model
    cfg = M.LLAMA3_8B
    t0 = 2048
    model = M.BitNetDecoder(cfg, seed=1, device=dev, dtype=torch.bfloat16, init_on_device=True,
                            backend=M.HipBackend(out_dtype=torch.bfloat16, fused=True))
    prompt = torch.randint(0, cfg.vocab_size, (BATCH, t0), generator=torch.Generator().manual_seed(9)).to(dev)
    new = 4
    eager = model.generate(prompt, new).cpu()
    graph = model.generate(prompt, new, graph=True).cpu()
    print("llama3-8b 8 x 2048: fused eager / graph done", flush=True)
    assert torch.equal(eager, graph), "graph replays diverge from eager decoding"

    Sampled = type("Sampled", (_SampledChecks, M.HipBackend), {})
    be = Sampled(out_dtype=torch.bfloat16, fused=False)
    be.setup(pkg, {id(l): n for n, l in M.quantised_linears(model).items()}, np.random.default_rng(1))
    model.backend = be
    projs = ("q", "k", "v", "o", "gate", "up", "down")
    with torch.no_grad():
        model.reset(BATCH, t0 + new)
        be.sample = {f"layers.0.{p}" for p in projs} | {"lm_head"}
        nxt = model.forward(prompt, 0, tokens=True)
        print(f"llama3-8b 8 x 2048: prefill checks {len(be.done)}", flush=True)
        toks = [nxt]
        ids = nxt[:, None].clone()
        pos = torch.full((BATCH,), t0, dtype=torch.long, device=dev)
        for s in range(new - 1):
            be.sample = ({f"layers.31.{p}" for p in projs} | {"lm_head"}) if s == 1 else set()
            nxt = model.decode_step(ids, pos, tokens=True)
            toks.append(nxt)
            ids = nxt[:, None].clone()
            pos += 1
    unfused = torch.stack(toks, dim=1).cpu()
    assert set(be.done) == {(p, BATCH * t0) for p in projs} | {(p, BATCH) for p in projs} | {("lm_head", BATCH)}
    assert torch.equal(unfused, eager), "unfused launches give different tokens from the fused path"
