"""Benchmark: GradDotProd on GPT-2-small, T=1024 on one MI355X.

A step is one GradDotProd training step of the reference's loop
(Examples/GradDotProd_LM/training_loop.py:99-166): forward on the concatenated 16 train + 4
val rows, backward with the dot-product hooks, .grad <- train grads, AdamW step, aggregate
and log the per-train-row dot vector (with its device->host copy), clear.  Inputs are
synthetic token ids already resident in HBM; weights are random N(0, 0.02), bf16.

Prints one JSON line: samples/s (train rows scored per second; the dot kernels run on a
side stream overlapped with the rest of backward), step overhead versus plain backprop of
the same batch, the roofline of the dominant hot-path op (timed with HIP events on the
stream it runs on, in a second pass of the same steps with the dot kernels serialised on
the autograd stream so that each op's time is its own), the fused ghost kernel at the
Linear microbench shape against the bf16 MFMA peak, and a CPU
baseline (the oracle's reference op sequence on the host cores).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_BF16 = 2.5e15   # MI355X dense bf16 MFMA, FLOP/s
PEAK_HBM = 8.0e12    # MI355X HBM3E, B/s
METRIC = "samples/sec w/ ghost dot-products, GPT-2-small T=1024; MFMA util %; step overhead"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


# ------------------------------------------------------------------ op timing
class TimedOps:
    """Wraps the kernel layer: brackets every call with HIP events on the current stream
    and records (op, algorithm, algorithmic work, events)."""

    def __init__(self, inner):
        self.inner = inner
        self.records = []
        self.enabled = False

    def _run(self, name, work, fn, *a, **k):
        if not self.enabled:
            return fn(*a, **k)
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record()
        out = fn(*a, **k)
        e.record()
        self.records.append((name, work, s, e))
        return out

    def __getattr__(self, name):
        # entry points without their own timing pass straight through
        return getattr(self.inner, name)

    def linear_algo(self, *a, **k):
        return self.inner.linear_algo(*a, **k)

    def embedding_train_grad(self, ids, G, n_val, scale, out, **k):
        # train rows of G and their ids, plus the table rows written: every row (overwrite),
        # or read + written for at most one row per train token (accumulate)
        n_tok = (G.shape[0] - n_val) * (ids.numel() // G.shape[0])
        row = out.shape[-1] * out.element_size()
        rows = 2 * min(out.shape[0], n_tok) if k.get("accumulate") else out.shape[0]
        nbytes = n_tok * (G.shape[-1] * G.element_size() + 8) + rows * row
        return self._run("embedding_train_grad", ("hbm", nbytes),
                         self.inner.embedding_train_grad, ids, G, n_val, scale, out, **k)

    def linear_dot(self, A, G, n_val, **k):
        from ghostsuite_amd import _native
        N, d_in, d_out = A.shape[0], A.shape[-1], G.shape[-1]
        T = A.numel() // (N * d_in)
        sem = k.get("semantics", 0)
        algo = self.inner.linear_algo(A.dtype, N, n_val, T, d_in, d_out, sem,
                                      k.get("algo", 0), k.get("want_pair", False))
        n_t = N - n_val
        nv = n_val if sem == _native.SEM_PAIRWISE_SUM else 1
        if algo == _native.ALGO_GHOST:
            flops = 2.0 * n_t * nv * T * T * (d_in + d_out)
        else:
            flops = 2.0 * (nv * T + n_t * T) * d_in * d_out
        name = f"linear_{_native.ALGO_NAMES[algo]}[{d_in}x{d_out}]"
        return self._run(name, ("mfma", flops), self.inner.linear_dot, A, G, n_val, **k)

    def linear_bias_dot(self, A, G, n_val, **k):
        from ghostsuite_amd import _native
        N, d_in, d_out = A.shape[0], A.shape[-1], G.shape[-1]
        T = A.numel() // (N * d_in)
        nv = n_val if k.get("semantics", 0) == _native.SEM_PAIRWISE_SUM else 1
        flops = 2.0 * (nv * T + (N - n_val) * T) * d_in * d_out
        out = self._run(f"linear_valgrad+bias[{d_in}x{d_out}]", ("mfma", flops),
                        self.inner.linear_bias_dot, A, G, n_val, **k)
        if out is None and self.enabled:
            self.records.pop()   # not supported for this shape: nothing ran
        return out

    def linear_dot_train_grad(self, A, G, n_val, **k):
        # The op's work is the dots by the cheapest same-semantics algorithm,
        # 2 (n_v' + n_t) T d_in d_out (the V GEMM over the val rows, then one GEMM over the
        # train rows), which is also what it executes: the weight train gradient is the
        # running sum of the same per-sample products, so it adds no flops.  What the two
        # outputs would cost apart (+ 2 n_t T d_in d_out) is kept only as a side figure.
        from ghostsuite_amd import _native
        N, d_in, d_out = A.shape[0], A.shape[-1], G.shape[-1]
        T = A.numel() // (N * d_in)
        nv = n_val if k.get("semantics", 0) == _native.SEM_PAIRWISE_SUM else 1
        dot = 2.0 * (nv * T + (N - n_val) * T) * d_in * d_out
        grad = 2.0 * (N - n_val) * T * d_in * d_out if k.get("grad_scale") is not None else 0.0
        tag = "+bias" if k.get("bias") else ""
        kind = "conv1d" if k.get("conv1d") else "linear"
        out = self._run(f"{kind}_valgrad{tag}+train_grad[{d_in}x{d_out}]",
                        ("mfma", dot, dot + grad),
                        self.inner.linear_dot_train_grad, A, G, n_val, **k)
        if out is None and self.enabled:
            self.records.pop()   # not supported for this shape: nothing ran
        return out

    def linear_train_grad(self, A, G, n_val, scale, **k):
        N, d_in, d_out = A.shape[0], A.shape[-1], G.shape[-1]
        T = A.numel() // (N * d_in)
        flops = 2.0 * (N - n_val) * T * d_in * d_out
        out = self._run(f"linear_train_grad[{d_in}x{d_out}]", ("mfma", flops),
                        self.inner.linear_train_grad, A, G, n_val, scale, **k)
        if out is None and self.enabled:
            self.records.pop()   # not taken by the kernel: the sampler's addmm runs instead
        return out

    def bias_dot(self, G, n_val, **k):
        return self._run("bias_dot", ("hbm", G.numel() * G.element_size()),
                         self.inner.bias_dot, G, n_val, **k)

    def embedding_dot(self, ids, G, n_val, vocab, **k):
        nbytes = G.numel() * G.element_size() + ids.numel() * 8
        return self._run("embedding_dot", ("hbm", nbytes), self.inner.embedding_dot, ids, G,
                         n_val, vocab, **k)

    def layernorm_dot(self, X, G, n_val, eps, **k):
        nbytes = X.numel() * X.element_size() + G.numel() * G.element_size()
        return self._run("layernorm_dot", ("hbm", nbytes), self.inner.layernorm_dot, X, G,
                         n_val, eps, **k)

    def kron_proj(self, A, G, P_i, P_o, scale, **k):
        nbytes = A.numel() * A.element_size() + G.numel() * G.element_size()
        return self._run("kron_proj", ("hbm", nbytes), self.inner.kron_proj, A, G, P_i, P_o,
                         scale, **k)

    def kron_embed_proj(self, ids, G, P_iT, P_o, scale=1.0, **k):
        nbytes = G.numel() * G.element_size() + ids.numel() * 8
        return self._run("kron_embed_proj", ("hbm", nbytes), self.inner.kron_embed_proj, ids,
                         G, P_iT, P_o, scale, **k)

    def summary(self):
        torch.cuda.synchronize()
        agg = {}
        for name, w, s, e in self.records:
            bound, work = w[0], w[1]
            ms = s.elapsed_time(e)
            a = agg.setdefault(name, {"bound": bound, "work": work, "ms": 0.0, "n": 0,
                                      "apart": w[2] if len(w) > 2 else work})
            a["ms"] += ms
            a["n"] += 1
        return agg


# ------------------------------------------------------------------ GPT-2-small step
def gpt2_bench(steps: int, warmup: int, dev):
    from ghostsuite_amd import GradDotProdEngine, _native
    from ghostsuite_amd import supported_layers_grad_samplers_dotprod as S
    from ghostsuite_amd.workloads import CausalLM, GPT2_SMALL, synthetic_tokens

    n_train, n_val, T = 16, 4, 1024
    cfg = GPT2_SMALL
    torch.manual_seed(0)
    model = CausalLM(cfg).to(dev, torch.bfloat16)
    plain = CausalLM(cfg).to(dev, torch.bfloat16)
    plain.load_state_dict(model.state_dict())
    X, Y = synthetic_tokens(n_train + n_val, T, cfg.vocab, seed=1234, device=dev)
    X_tr, Y_tr = X[:n_train], Y[:n_train]

    timed = TimedOps(_native.ops())
    _native._install_backend(timed)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-4)
    engine = GradDotProdEngine(model, val_batch_size=n_val, loss_reduction="mean",
                               use_dummy_bias=True, record_algorithms=True)
    engine.attach(opt)

    def ghost_step(i):
        engine.attach_train_batch(X_tr, Y_tr, i, 0)
        loss = model(X, Y)
        loss.backward()
        engine.prepare_gradients()
        opt.step()
        engine.aggregate_and_log()
        engine.clear_gradients()
        opt.zero_grad(set_to_none=True)
        engine.dot_product_log.clear()

    popt = torch.optim.AdamW(plain.parameters(), lr=1e-4)

    def plain_step(i):
        loss = plain(X, Y)
        loss.backward()
        popt.step()
        popt.zero_grad(set_to_none=True)

    def run(fn, n_steps, n_warm, label):
        for i in range(n_warm):
            fn(i)
        torch.cuda.synchronize()
        log(f"[bench] {label}: warmup done, timing {n_steps} steps")
        t0 = time.perf_counter()
        for i in range(n_steps):
            fn(i)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n_steps

    # Throughput: the dot kernels overlap the rest of backward on a side stream.
    timed.enabled = False
    t_ghost = run(ghost_step, steps, warmup, "ghost")
    log(f"[bench] ghost step {t_ghost * 1e3:.2f} ms")
    # Per-op breakdown: the same steps with the dot kernels serialised on the autograd
    # stream, each op bracketed by HIP events, so that an op's time is its own.
    S.options["overlap"] = False
    timed.enabled = True
    t0 = time.perf_counter()
    for i in range(steps):
        ghost_step(i)
    torch.cuda.synchronize()
    t_serial = (time.perf_counter() - t0) / steps
    timed.enabled = False
    S.options["overlap"] = True
    ops_summary = timed.summary()
    log(f"[bench] ghost step, serialised dot kernels: {t_serial * 1e3:.2f} ms")
    t_plain = run(plain_step, steps, warmup, "plain")
    log(f"[bench] plain step {t_plain * 1e3:.2f} ms")

    def plain_train_step(i):   # plain backprop of the n_train rows only
        loss = plain(X_tr, Y_tr)
        loss.backward()
        popt.step()
        popt.zero_grad(set_to_none=True)

    t_plain_train = run(plain_train_step, steps, warmup, "plain (train rows only)")
    _native._install_backend(None)
    engine.detach()
    algos = dict(S.ALGO_LOG)
    del model, plain, opt, popt, engine
    torch.cuda.empty_cache()
    return {
        "n_train": n_train, "n_val": n_val, "T": T,
        "t_ghost": t_ghost, "t_serial": t_serial, "t_plain": t_plain,
        "t_plain_train": t_plain_train, "ops": ops_summary,
        "algos": algos,
        "plain_tflop": __import__("ghostsuite_amd.workloads", fromlist=["x"]).lm_flops_per_step(
            cfg, n_train + n_val, T) / 1e12,
    }


# ------------------------------------------------------------------ GradProj
def gradproj_bench(steps: int, warmup: int, dev):
    """GPT-2-medium shape, B=32, T=1024, bf16; Kronecker projection k_i = k_o = 16 on every
    block Linear (96 layers); per step: forward, backward, collect_batch (fp16), async copy of
    the projections to pinned host memory.  Ends with the pairwise similarity proj @ proj^T."""
    from ghostsuite_amd import _native
    from ghostsuite_amd.gradProjection.gradproj_engine import GradProjLoraEngine
    from ghostsuite_amd.workloads import CausalLM, GPT2_MEDIUM, synthetic_tokens
    import tempfile
    B, T = 32, 1024
    torch.manual_seed(0)
    model = CausalLM(GPT2_MEDIUM).to(dev, torch.bfloat16)
    X, Y = synthetic_tokens(B, T, GPT2_MEDIUM.vocab, seed=77, device=dev)
    timed = TimedOps(_native.ops())
    _native._install_backend(timed)
    tmp = tempfile.mkdtemp()
    eng = GradProjLoraEngine(model, proj_layers="h.", proj_rank_total=256, proj_rank_min=8,
                             proj_seed=42, proj_dtype="float16", proj_dir=tmp,
                             proj_save_interval=10 ** 9, proj_dims_override=(16, 16))
    eng.attach()
    host = torch.empty((B, eng.total_proj_dim), dtype=torch.float16, pin_memory=True)

    def step():
        model.zero_grad(set_to_none=True)
        loss = model(X, Y)
        loss.backward()
        proj = eng.collect_batch()
        host.copy_(proj, non_blocking=True)
        eng.clear_gradients()
        return proj

    from ghostsuite_amd import _overlap

    def timed_steps(fn):
        t0 = time.perf_counter()
        out = None
        for _ in range(steps):
            out = fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps, out

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t, proj = timed_steps(step)   # projection kernels overlapped on the side stream
    # Per-op pass: kernels serialised on the autograd stream, each bracketed by HIP events.
    _overlap.enabled = False
    timed.enabled = True
    timed_steps(step)
    timed.enabled = False
    _overlap.enabled = True
    sim = (proj.float() @ proj.float().t()).cpu()
    ops = timed.summary()
    _native._install_backend(None)
    eng.detach()

    def plain_step():
        model.zero_grad(set_to_none=True)
        model(X, Y).backward()

    for _ in range(warmup):
        plain_step()
    torch.cuda.synchronize()
    t_plain, _ = timed_steps(plain_step)
    kp = ops.get("kron_proj", {"ms": 0.0, "n": 1, "work": 0})
    avg = kp["ms"] / max(kp["n"], 1)
    # MFMA work of the projections: 2*B*T*(n_a*k_i + n_g*k_o) per layer (the outer products
    # over tokens add 2*B*T*k_i*k_o), summed over the 96 layers of one step.
    cfgm = GPT2_MEDIUM
    kf = 0.0
    dm, dff = cfgm.d_model, cfgm.d_mlp
    for n_a, n_g in ((dm, 3 * dm), (dm, dm), (dm, dff), (dff, dm)):
        kf += cfgm.n_layer * 2.0 * B * T * (16 * n_a + 16 * n_g + 16 * 16)
    bytes_per_step = kp["work"] * kp["n"] / steps if kp["n"] else 0
    del model, eng
    torch.cuda.empty_cache()
    return {"workload": "GPT-2-medium shape GradProj, B=32, T=1024, k=16x16 on 96 Linear layers",
            "ms_per_step": t * 1e3, "samples_per_s": B / t,
            "plain_ms_per_step": t_plain * 1e3, "step_overhead": t / t_plain,
            "proj_dim": int(host.shape[1]), "similarity_finite": bool(torch.isfinite(sim).all()),
            "kron_ms_per_step": kp["ms"] / steps, "kron_calls_per_step": kp["n"] / steps,
            "kron_avg_us": avg * 1e3,
            "kron_hbm_GBps": (bytes_per_step / (kp["ms"] / steps * 1e-3) / 1e9) if kp["ms"] else None,
            "kron_hbm_frac": (bytes_per_step / (kp["ms"] / steps * 1e-3) / PEAK_HBM) if kp["ms"] else None,
            "kron_mfma_TFLOPs": (kf / (kp["ms"] / steps * 1e-3) / 1e12) if kp["ms"] else None,
            "kron_mfma_frac": (kf / (kp["ms"] / steps * 1e-3) / 2.5e15) if kp["ms"] else None}


# ------------------------------------------------------------------ Pythia-1B shape
def pythia_bench(steps: int, warmup: int, dev):
    """16 layers, d=2048, MLP 8192, T=2048, rotary, untied embed_out, bf16; 8 train + 2 val."""
    from ghostsuite_amd import GradDotProdEngine, _native
    from ghostsuite_amd import supported_layers_grad_samplers_dotprod as S
    from ghostsuite_amd.workloads import CausalLM, PYTHIA_1B, synthetic_tokens
    n_train, n_val, T = 8, 2, 2048
    torch.manual_seed(0)
    model = CausalLM(PYTHIA_1B).to(dev, torch.bfloat16)
    plain = CausalLM(PYTHIA_1B).to(dev, torch.bfloat16)
    plain.load_state_dict(model.state_dict())
    X, Y = synthetic_tokens(n_train + n_val, T, PYTHIA_1B.vocab, seed=99, device=dev)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-4)
    eng = GradDotProdEngine(model, val_batch_size=n_val, use_dummy_bias=True)
    eng.attach(opt)
    popt = torch.optim.AdamW(plain.parameters(), lr=1e-4)

    def ghost_step(i):
        eng.attach_train_batch(X[:n_train], Y[:n_train], i, 0)
        model(X, Y).backward()
        eng.prepare_gradients()
        opt.step()
        eng.aggregate_and_log()
        eng.clear_gradients()
        opt.zero_grad(set_to_none=True)
        eng.dot_product_log.clear()

    def plain_step(i):
        plain(X, Y).backward()
        popt.step()
        popt.zero_grad(set_to_none=True)

    timed = TimedOps(_native.ops())
    _native._install_backend(timed)

    def timed_run(fn):
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(steps):
            fn(i)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps

    out = {"ghost": timed_run(ghost_step)}
    # Per-op pass: dot kernels serialised on the autograd stream, bracketed by HIP events.
    S.options["overlap"] = False
    timed.enabled = True
    out["serial"] = timed_run(ghost_step)
    timed.enabled = False
    S.options["overlap"] = True
    ops = timed.summary()
    _native._install_backend(None)
    out["plain"] = timed_run(plain_step)
    eng.detach()
    del model, plain, opt, popt, eng
    torch.cuda.empty_cache()
    per_op = {}
    for name, a in sorted(ops.items(), key=lambda kv: -kv[1]["ms"]):
        calls = a["n"] / (steps + warmup)
        avg_ms = a["ms"] / a["n"]
        rate = a["work"] / (avg_ms * 1e-3)
        per_op[name] = {"ms_per_step": a["ms"] / (steps + warmup), "calls_per_step": calls,
                        "avg_us": avg_ms * 1e3,
                        ("TFLOP/s" if a["bound"] == "mfma" else "GB/s"): rate / 1e12
                        if a["bound"] == "mfma" else rate / 1e9}
    return {"workload": "Pythia-1B shape GradDotProd, 8 train + 2 val, T=2048",
            "ms_per_step": out["ghost"] * 1e3, "plain_ms_per_step": out["plain"] * 1e3,
            "ms_per_step_serialised_dots": out["serial"] * 1e3,
            "samples_per_s": n_train / out["ghost"], "step_overhead": out["ghost"] / out["plain"],
            "ops": per_op}


def hf_gpt2_bench(steps: int, warmup: int, dev):
    """The reference LM example's model: a Hugging Face GPT2LMHeadModel at the GPT-2-small
    configuration (HF Conv1D attention and MLP layers, tied head, dropout off), bf16, 16 train
    + 4 val rows at T=1024 with per-sample position ids, against plain backprop of the same
    model.  Random-init weights, synthetic ids."""
    import transformers
    from ghostsuite_amd import GradDotProdEngine, _native
    from ghostsuite_amd import supported_layers_grad_samplers_dotprod as S
    from ghostsuite_amd.workloads import synthetic_tokens
    n_train, n_val, T, vocab = 16, 4, 1024, 50257
    cfg = transformers.GPT2Config(n_layer=12, n_embd=768, n_head=12, vocab_size=vocab,
                                  n_positions=T, resid_pdrop=0.0, embd_pdrop=0.0,
                                  attn_pdrop=0.0)
    torch.manual_seed(0)
    model = transformers.GPT2LMHeadModel(cfg).eval().to(dev, torch.bfloat16)
    plain = transformers.GPT2LMHeadModel(cfg).eval().to(dev, torch.bfloat16)
    plain.load_state_dict(model.state_dict())
    X, _ = synthetic_tokens(n_train + n_val, T, vocab, seed=98, device=dev)
    pos = torch.arange(T, device=dev).expand(n_train + n_val, T).contiguous()
    opt = torch.optim.AdamW(model.parameters(), lr=1e-4)
    # The embeddings get the engine's dummy bias (as the reference's forward swapper gives
    # them), so that autograd skips every weight-gradient GEMM the hooks supply.
    model.ghost_embeddings = ["transformer.wte", "transformer.wpe"]
    eng = GradDotProdEngine(model, val_batch_size=n_val, use_dummy_bias=True)
    eng.attach(opt)
    popt = torch.optim.AdamW(plain.parameters(), lr=1e-4)

    def ghost_step(i):
        eng.attach_train_batch(X[:n_train], X[:n_train], i, 0)
        model(input_ids=X, position_ids=pos, labels=X).loss.backward()
        eng.prepare_gradients()
        opt.step()
        eng.aggregate_and_log()
        eng.clear_gradients()
        opt.zero_grad(set_to_none=True)
        eng.dot_product_log.clear()

    def plain_step(i):
        plain(input_ids=X, position_ids=pos, labels=X).loss.backward()
        popt.step()
        popt.zero_grad(set_to_none=True)

    timed = TimedOps(_native.ops())
    _native._install_backend(timed)

    def timed_run(fn):
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(steps):
            fn(i)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps

    out = {"ghost": timed_run(ghost_step)}
    S.options["overlap"] = False
    timed.enabled = True
    out["serial"] = timed_run(ghost_step)
    timed.enabled = False
    S.options["overlap"] = True
    ops = timed.summary()
    _native._install_backend(None)
    out["plain"] = timed_run(plain_step)
    eng.detach()
    del model, plain, opt, popt, eng
    torch.cuda.empty_cache()
    per_op = {}
    for name, a in sorted(ops.items(), key=lambda kv: -kv[1]["ms"]):
        avg_ms = a["ms"] / a["n"]
        rate = a["work"] / (avg_ms * 1e-3)
        per_op[name] = {"ms_per_step": a["ms"] / (steps + warmup),
                        "calls_per_step": a["n"] / (steps + warmup), "avg_us": avg_ms * 1e3,
                        ("TFLOP/s" if a["bound"] == "mfma" else "GB/s"): rate / 1e12
                        if a["bound"] == "mfma" else rate / 1e9}
    return {"workload": "Hugging Face GPT2LMHeadModel (GPT-2-small config, Conv1D layers) "
                        "GradDotProd step, 16 train + 4 val, T=1024",
            "ms_per_step": out["ghost"] * 1e3, "plain_ms_per_step": out["plain"] * 1e3,
            "ms_per_step_serialised_dots": out["serial"] * 1e3,
            "samples_per_s": n_train / out["ghost"], "step_overhead": out["ghost"] / out["plain"],
            "ops": per_op}


# ------------------------------------------------------------------ ghost kernel microbench
def timed_blocks(fn, warmup: int, reps: int, blocks: int):
    """`warmup` untimed calls of fn, then `blocks` timed blocks of `reps` calls on the current
    stream; returns (the median block's average ms per call, every block's average)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    block_ms = []
    for _ in range(blocks):
        s.record()
        for _ in range(reps):
            fn()
        e.record()
        torch.cuda.synchronize()
        block_ms.append(s.elapsed_time(e) / reps)
    return sorted(block_ms)[len(block_ms) // 2], block_ms


def ghost_kernel_bench(dev, reps: int = 20, T: int = 1024, warmup: int = 12, blocks: int = 5):
    """A[32,T,768], G[32,T,3072] bf16, first 8 rows val, fused ghost.

    `warmup` untimed calls, then `blocks` timed blocks of `reps` calls; `ms` is the median
    block's average (every block is reported).  The first dozen calls after other work run
    up to ~20% slower than the steady state while the chip's clock settles."""
    from ghostsuite_amd import _native
    g = torch.Generator().manual_seed(1234)
    N, n_val, d_in, d_out = 32, 8, 768, 3072
    A = torch.randn(N, T, d_in, generator=g).to(dev, torch.bfloat16)
    G = (torch.randn(N, T, d_out, generator=g) * 1e-3).to(dev, torch.bfloat16)
    ops = _native.ops()
    ms, block_ms = timed_blocks(
        lambda: ops.linear_dot(A, G, n_val, val_start=0, algo=_native.ALGO_GHOST),
        warmup, reps, blocks)
    flops = 2.0 * (N - n_val) * n_val * T * T * (d_in + d_out)
    # same semantics through the val-gradient algorithm, for reference
    ms_vg, _ = timed_blocks(
        lambda: ops.linear_dot(A, G, n_val, val_start=0, algo=_native.ALGO_VALGRAD),
        warmup, reps, 3)
    return {"T": T, "ms": ms, "tflops": flops / ms / 1e9, "frac": flops / (ms * 1e-3) / PEAK_BF16,
            "valgrad_ms": ms_vg, "block_ms": block_ms, "warmup_calls": warmup,
            "calls_per_block": reps}


def achievable_peak(dev, reps: int = 10, n: int = 8192, warmup: int = 12, blocks: int = 5):
    """The bf16 GEMM rate this box reaches with the vendor library: torch.mm (hipBLASLt) on
    n x n x n bf16 operands, beside the nominal dense peak (the clock falls under the power
    limit as MFMA activity rises, so no kernel reaches 2.5 PF/s).  Timed like the ghost
    kernel: `warmup` calls, then the median of `blocks` blocks of `reps` calls."""
    g = torch.Generator().manual_seed(11)
    a = torch.randn(n, n, generator=g).to(dev, torch.bfloat16)
    b = torch.randn(n, n, generator=g).to(dev, torch.bfloat16)
    ms, block_ms = timed_blocks(lambda: torch.mm(a, b), warmup, reps, blocks)
    del a, b
    return {"kernel": f"torch.mm (hipBLASLt) bf16 {n}x{n}x{n}", "ms": ms,
            "TFLOP/s": 2.0 * n ** 3 / (ms * 1e-3) / 1e12, "ms_per_block": block_ms}


def vendor_route(dev, reps: int = 10):
    """The dominant op's outputs at the fc_out shape (A[20,1024,3072], G[20,1024,768] bf16,
    4 val rows last) through the vendor library instead: V = G_val^T A_val, the row-dot
    GEMM A_train V^T with its per-sample reduction against G_train, and the train gradient
    G_train^T A_train (three torch.mm calls on hipBLASLt plus torch's elementwise reduction;
    the transposed operands made contiguous outside the timed region, except V^T)."""
    g = torch.Generator().manual_seed(21)
    N, n_val, T, d_in, d_out = 20, 4, 1024, 3072, 768
    n_t = N - n_val
    A = torch.randn(N * T, d_in, generator=g).to(dev, torch.bfloat16)
    G = (torch.randn(N * T, d_out, generator=g) * 1e-3).to(dev, torch.bfloat16)
    A_tr, A_v = A[: n_t * T], A[n_t * T:]
    G_tr = G[: n_t * T]
    G_vT = G[n_t * T:].t().contiguous()
    G_trT = G_tr.t().contiguous()

    def route():
        V = torch.mm(G_vT, A_v)                                   # [d_out, d_in]
        U = torch.mm(A_tr, V.t().contiguous())                    # [n_t T, d_out]
        dots = (U.float() * G_tr.float()).sum(1).view(n_t, T).sum(1)
        grad = torch.mm(G_trT, A_tr)                              # [d_out, d_in]
        return dots, grad

    for _ in range(3):
        route()
    torch.cuda.synchronize()
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        route()
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / reps
    del A, G, G_vT, G_trT
    return {"shape": "A[20,1024,3072] G[20,1024,768] bf16, 4 val rows last (fc_out)",
            "ms": ms, "kernels": "torch.mm (hipBLASLt) x3 + torch elementwise row-dot"}


def emb_grad_pad_bench(dev, reps: int = 10):
    """The Embedding train gradient on a padded batch: 32 train + 2 val rows of T=2048 with
    90% of the tokens one pad id (65536 train tokens, a 59k-token run), d=768, vocab 50257,
    bf16, both modes; against the same call on uniform ids of the same shape."""
    from ghostsuite_amd import _native
    g = torch.Generator().manual_seed(5)
    N, n_val, T, d, V = 34, 2, 2048, 768, 50257
    ids = torch.randint(0, V, (N, T), generator=g)
    ids_pad = ids.clone()
    ids_pad[torch.rand(N, T, generator=g) < 0.9] = V - 1
    G = (torch.randn(N, T, d, generator=g) * 1e-2).to(dev, torch.bfloat16)
    tab = torch.zeros(V, d, dtype=torch.bfloat16, device=dev)
    ops = _native.ops()
    out = {}
    for name, x in (("padded", ids_pad.to(dev)), ("uniform", ids.to(dev))):
        for acc in (False, True):
            fn = lambda: ops.embedding_train_grad(x, G, n_val, 1.0, tab, accumulate=acc)
            fn()
            torch.cuda.synchronize()
            s = torch.cuda.Event(enable_timing=True)
            e = torch.cuda.Event(enable_timing=True)
            s.record()
            for _ in range(reps):
                fn()
            e.record()
            torch.cuda.synchronize()
            out[f"{name}_{'accumulate' if acc else 'overwrite'}_us"] = s.elapsed_time(e) / reps * 1e3
    del G, tab
    return {"shape": "ids[34,2048] (32 train + 2 val rows), G[34,2048,768] bf16, vocab 50257",
            **out}


def ghost_sweep(dev, reps: int = 6, warmup: int = 6, blocks: int = 3):
    """BASELINE configs[1] sweep over T: the reference's switch (2T^2 <= d_in*d_out) picks the
    ghost (pairwise-sum) branch up to T=1024 and the materialised (presum) branch at T=2048;
    each semantics is timed with both algorithms (timed_blocks: the median block)."""
    from ghostsuite_amd import _native
    g = torch.Generator().manual_seed(1234)
    N, n_val, d_in, d_out = 32, 8, 768, 3072
    ops = _native.ops()
    out = []
    for T in (128, 512, 1024, 2048):
        A = torch.randn(N, T, d_in, generator=g).to(dev, torch.bfloat16)
        G = (torch.randn(N, T, d_out, generator=g) * 1e-3).to(dev, torch.bfloat16)
        ghost_branch = 2 * T * T <= d_in * d_out
        sem = _native.SEM_PAIRWISE_SUM if ghost_branch else _native.SEM_PRESUM
        row = {"T": T, "reference_branch": "ghost" if ghost_branch else "materialised",
               "semantics": "pairwise" if ghost_branch else "presum"}
        for algo, name in ((_native.ALGO_GHOST, "ghost"), (_native.ALGO_VALGRAD, "valgrad")):
            fn = lambda: ops.linear_dot(A, G, n_val, val_start=0, semantics=sem, algo=algo)
            row[f"{name}_ms"], _ = timed_blocks(fn, warmup, reps, blocks)
        n_t, nv = N - n_val, (n_val if ghost_branch else 1)
        ghost_flops = 2.0 * n_t * nv * T * T * (d_in + d_out)
        row["ghost_TFLOPs"] = ghost_flops / row["ghost_ms"] / 1e9
        row["auto"] = _native.ALGO_NAMES[ops.linear_algo(torch.bfloat16, N, n_val, T, d_in,
                                                          d_out, sem, _native.ALGO_AUTO, False)]
        out.append(row)
        del A, G
    return out


# ------------------------------------------------------------------ CPU baseline
def _cpu_model() -> str:
    """The host CPU as /proc/cpuinfo names it, with its family / model numbers (a
    virtualised host may report only the brand) and the logical CPUs the OS shows."""
    fields = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                key, _, val = line.partition(":")
                key = key.strip()
                if key in ("model name", "cpu family", "model") and key not in fields:
                    fields[key] = val.strip()
                if len(fields) == 3:
                    break
    except OSError:
        pass
    name = fields.get("model name", "unknown")
    if "cpu family" in fields and "model" in fields:
        name += f" (family {fields['cpu family']}, model {fields['model']})"
    return f"{name}, {os.cpu_count()} logical CPUs on the host"


def cpu_baseline(budget_s: float = 60.0):
    """One whole GPT-2-small GradDotProd step (16 train + 4 val rows, T=1024, bf16) through
    the reference's op sequence on the host cores, timed end to end: the oracle's
    restatement of every hooked sampler at full size (dots and train gradients of the 48
    block Linear layers and 25 LayerNorms, wte and wpe, and the tied lm_head's ghost dot,
    which the reference computes before wte overwrites it) plus the model's forward and
    input-gradient backward on all 20 rows (the reference freezes the weights and supplies
    their gradients from the hooks).  The block samplers run on one block's activations
    twelve times over (the work per block is the same).  Reported as train rows per
    second.  ``budget_s`` bounds the run: past it the remaining parts are skipped and the
    result says so."""
    from oracle import ghost_ref as R
    from ghostsuite_amd.workloads import CausalLM, GPT2_SMALL, synthetic_tokens
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    N, n_val, T, d, m, V = 20, 4, 1024, 768, 3072, GPT2_SMALL.vocab
    n_t = N - n_val
    g = torch.Generator().manual_seed(0)
    bf = torch.bfloat16

    def rnd(*shape, s=1.0):
        return (torch.randn(*shape, generator=g) * s).to(bf)

    layers = [("qkv", d, 3 * d), ("proj", d, d), ("fc", d, m), ("fc_out", m, d)]
    acts = {n: (rnd(N, T, a), rnd(N, T, b, s=1e-3)) for n, a, b in layers}
    ln_in, ln_g = rnd(N, T, d), rnd(N, T, d, s=1e-3)
    ids = torch.randint(0, V, (N, T), generator=g)
    pos = torch.arange(T).repeat(N, 1)
    A_lm, B_lm = rnd(N, T, d), rnd(N, T, V, s=1e-4)
    torch.manual_seed(0)
    model = CausalLM(GPT2_SMALL).to(bf)
    for p in model.parameters():
        p.requires_grad_(False)
    X, Y = synthetic_tokens(N, T, V, seed=3)

    def one_block():
        for name, a, b in layers:
            A, B = acts[name]
            R.linear_dot_ref(A, B, n_val, R.should_use_ghost(T, a * b))
            R.linear_train_grad(A, B * N, n_val)
        for _ in range(2):
            R.layernorm_dot_ref(ln_in, ln_g, n_val, 1e-5)
            R.layernorm_train_grad(ln_in, ln_g * N, n_val, 1e-5)

    def embeddings_and_ln_f():
        for x, vocab in ((ids, V), (pos, T)):
            R.embedding_dot_ref(x, ln_g, n_val, vocab)
            R.embedding_train_grad(x, ln_g * N, n_val, (vocab, d))
        R.layernorm_dot_ref(ln_in, ln_g, n_val, 1e-5)
        R.layernorm_train_grad(ln_in, ln_g * N, n_val, 1e-5)

    def lm_head():   # the tied lm_head: ghost branch (2 T^2 <= V d), no bias; train grad
        R.linear_dot_ref(A_lm, B_lm, n_val, True, has_bias=False)
        R.linear_train_grad(A_lm, B_lm * N, n_val)

    def fwd_bwd():
        x = model.wte(X).detach().requires_grad_(True)   # the dummy bias's role: a graph
        h = x + model.wpe(torch.arange(T).repeat(N, 1))
        for blk in model.h:
            h = blk(h)
        logits = model.lm_head(model.ln_f(h))
        loss = torch.nn.functional.cross_entropy(logits.float().view(-1, V), Y.reshape(-1))
        loss.backward()

    one_block()   # first-call allocations of the sampler sequence, not timed
    parts, skipped = {}, []
    plan = [("block_samplers", one_block, 12), ("embeddings_ln_f", embeddings_and_ln_f, 1),
            ("lm_head_dot_and_grad", lm_head, 1), ("model_fwd_bwd", fwd_bwd, 1)]
    t_all = time.perf_counter()
    for name, fn, reps in plan:
        t0 = time.perf_counter()
        for _ in range(reps):
            if time.perf_counter() - t_all > budget_s:
                skipped.append(name)
                break
            fn()
        parts[name] = time.perf_counter() - t0
    t_step = time.perf_counter() - t_all
    # The Linear microbench (configs[1], T=1024: A[32,1024,768], G[32,1024,3072] bf16, 8 val
    # rows), the reference's ghost branch on the same cores, once, if the budget allows.
    micro = None
    if time.perf_counter() - t_all < budget_s:
        del acts, A_lm, B_lm, model
        A_mb, G_mb = rnd(32, 1024, 768), rnd(32, 1024, 3072, s=1e-3)
        t0 = time.perf_counter()
        R.linear_dot_ref(A_mb, G_mb, 8, True, has_bias=False)
        micro = {"shape": "A[32,1024,768] G[32,1024,3072] bf16, 8 val rows, ghost branch",
                 "s": time.perf_counter() - t0}
    return {"value": n_t / t_step, "unit": "samples/s", "cores": threads, "kind": "port",
            "ghost_microbench": micro,
            "cpu_model": _cpu_model(), "s_per_step": t_step,
            "s_per_step_parts": {k: round(v, 3) for k, v in parts.items()},
            "complete": not skipped, "skipped": skipped,
            "sample": ("one whole step timed end to end: the oracle's restatement of the "
                       "reference's op sequence (torch CPU, bf16) for every hooked sampler of "
                       "GPT-2-small at 16+4 rows, T=1024 (12 blocks' 4 Linear + 2 LayerNorm "
                       "samplers, wte, wpe, ln_f, the tied lm_head's ghost dot and train "
                       "grad on all rows) and the model's forward + input-gradient backward "
                       "on all 20 rows")}


KERNEL_SHAPES = {
    # name: shape at which the kernel leg runs it (the GPT-2-small / GPT-2-medium bench shapes)
    "ghost_microbench": "linear_dot GHOST, A[32,1024,768] G[32,1024,3072] bf16, 8 val first",
    "valgrad_fc": "linear_dot VALGRAD pairwise, A[20,1024,768] G[20,1024,3072] bf16, 4 val",
    "valgrad_bias_fc": "linear_bias_dot (weight + bias dots, bias grad), A[20,1024,768] "
                       "G[20,1024,3072] bf16, 4 val",
    "valgrad_bias_fc_out": "linear_bias_dot (weight + bias dots, bias grad), A[20,1024,3072] "
                           "G[20,1024,768] bf16, 4 val",
    "valgrad_bias_qkv": "linear_bias_dot presum (weight + bias dots, bias grad), A[20,1024,768] "
                        "G[20,1024,2304] bf16, 4 val",
    "valgrad_bias_proj": "linear_bias_dot presum (weight + bias dots, bias grad), "
                         "A[20,1024,768] G[20,1024,768] bf16, 4 val",
    "dot_train_grad_fc": "linear_dot_train_grad (weight + bias dots, weight + bias train "
                         "grads), A[20,1024,768] G[20,1024,3072] bf16, 4 val",
    "dot_train_grad_fc_out": "linear_dot_train_grad (weight + bias dots and train grads), "
                             "A[20,1024,3072] G[20,1024,768] bf16, 4 val",
    "dot_train_grad_qkv": "linear_dot_train_grad presum (weight + bias dots and train grads), "
                          "A[20,1024,768] G[20,1024,2304] bf16, 4 val",
    "dot_train_grad_proj": "linear_dot_train_grad presum (weight + bias dots and train grads), "
                           "A[20,1024,768] G[20,1024,768] bf16, 4 val",
    "train_grad_fc": "linear_train_grad (fc weight's train gradient), A[20,1024,768] "
                     "G[20,1024,3072] bf16, 16 train rows",
    "train_grad_proj": "linear_train_grad (proj weight's train gradient), A[20,1024,768] "
                       "G[20,1024,768] bf16, 16 train rows",
    "bias_fc": "bias_dot, G[20,1024,3072] bf16, 4 val",
    "layernorm": "layernorm_dot + grads, X,G[20,1024,768] bf16, 4 val",
    "embedding_wte": "embedding_dot, ids[20,1024] vocab 50257, G[20,1024,768] bf16, 4 val",
    "embedding_grad_tied": "embedding_train_grad accumulate (into a tied lm_head grad), "
                           "ids[20,1024] vocab 50257, G[20,1024,768] bf16, 4 val",
    "embedding_grad_untied": "embedding_train_grad overwrite (every row written), ids[20,1024] "
                             "vocab 50257, G[20,1024,768] bf16, 4 val",
    "dot_train_grad_conv1d_c_fc": "conv1d_dot_train_grad presum (HF Conv1D c_fc: weight + bias "
                                  "dots and train grads), A[20,1024,768] G[20,1024,3072] bf16, "
                                  "4 val",
    "dot_train_grad_conv1d_c_attn": "conv1d_dot_train_grad presum (HF Conv1D c_attn), "
                                    "A[20,1024,768] G[20,1024,2304] bf16, 4 val",
    "embedding_grad_padded": "embedding_train_grad overwrite, ids[34,2048] with 90% one pad id "
                             "(65536 train tokens), vocab 50257, G[34,2048,768] bf16, 2 val",
    "train_grad_lm_head_hipblaslt": "torch.addmm (hipBLASLt): the GPT-2 tied lm_head's train "
                                    "gradient [50257,768] from 16 train rows of T=1024 (50257 "
                                    "columns: rows not 16-byte aligned for the K-major kernel)",
    "train_grad_pythia_fc": "linear_train_grad (256x256-tile K-major kernel), A[10,2048,2048] "
                            "G[10,2048,8192] bf16, 8 train rows",
    "train_grad_pythia_fc_hipblaslt": "torch.addmm (hipBLASLt) at the same shape",
    "kron_fc": "kron_proj, A[32,1024,1024] G[32,1024,4096] bf16, k=16x16",
    "kron_embed_wte": "kron_embed_proj, ids[32,1024] vocab 50257, G[32,1024,1024] bf16, k=16x16",
    "copy_1GiB": "device copy of 1 GiB (HBM calibration)",
}


def kernels_leg(dev, reps: int = 10, warmup: int = 4):
    """Kernel-level leg for counter runs: every hot-path entry point at its bench shape,
    `warmup` untimed calls (12 for the ghost kernel, which runs first, while the clock
    settles) and `reps` timed ones, plus a 1 GiB device copy (the calibration for FETCH_SIZE
    and WRITE_SIZE).  Prints one JSON line of average milliseconds per call."""
    from ghostsuite_amd import _native
    ops = _native.ops()
    g = torch.Generator().manual_seed(7)

    def rnd(*shape, s=1.0):
        return (torch.randn(*shape, generator=g) * s).to(dev, torch.bfloat16)

    # One-element ops bracket each entry point in kernel traces and counter dumps: a
    # bitwise_not before its first call and a neg after its last (entries in the order of
    # the printed JSON line).
    marker = torch.zeros(1, dtype=torch.int32, device=dev)

    def timeit(fn, warm=warmup):
        marker.bitwise_not_()
        for _ in range(warm):
            fn()
        torch.cuda.synchronize()
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            fn()
        e.record()
        marker.neg_()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / reps

    out = {}
    A = rnd(32, 1024, 768)
    G = rnd(32, 1024, 3072, s=1e-3)
    out["ghost_microbench"] = timeit(lambda: ops.linear_dot(A, G, 8, val_start=0,
                                                           algo=_native.ALGO_GHOST), warm=12)
    A2, G2 = A[:20].contiguous(), G[:20].contiguous()
    out["valgrad_fc"] = timeit(lambda: ops.linear_dot(A2, G2, 4, algo=_native.ALGO_VALGRAD))
    out["valgrad_bias_fc"] = timeit(lambda: ops.linear_bias_dot(A2, G2, 4,
                                                                algo=_native.ALGO_VALGRAD,
                                                                grad_scale=1.25))
    for key, a_src, g_src, sem in (
            ("valgrad_bias_fc_out", G2, A2, _native.SEM_PAIRWISE_SUM),
            ("valgrad_bias_qkv", A2, G2[..., :2304], _native.SEM_PRESUM),
            ("valgrad_bias_proj", A2, A2, _native.SEM_PRESUM)):
        a_op, g_op = a_src.contiguous(), (g_src * 1e-3 if g_src is A2 else g_src).contiguous()
        out[key] = timeit(lambda: ops.linear_bias_dot(a_op, g_op, 4, semantics=sem,
                                                      algo=_native.ALGO_VALGRAD,
                                                      grad_scale=1.25))
        del a_op, g_op
    for key, a_src, g_src, sem in (
            ("dot_train_grad_fc", A2, G2, _native.SEM_PAIRWISE_SUM),
            ("dot_train_grad_fc_out", G2, A2, _native.SEM_PAIRWISE_SUM),
            ("dot_train_grad_qkv", A2, G2[..., :2304], _native.SEM_PRESUM),
            ("dot_train_grad_proj", A2, A2, _native.SEM_PRESUM)):
        a_op, g_op = a_src.contiguous(), (g_src * 1e-3 if g_src is A2 else g_src).contiguous()
        out[key] = timeit(lambda: ops.linear_dot_train_grad(
            a_op, g_op, 4, semantics=sem, grad_scale=1.25 / 16, bias=True,
            bias_grad_scale=1.25 / 16))
        del a_op, g_op
    out["train_grad_fc"] = timeit(lambda: ops.linear_train_grad(A2, G2, 4, 1.25 / 16))
    GP = (A2 * 1e-3).contiguous()
    out["train_grad_proj"] = timeit(lambda: ops.linear_train_grad(A2, GP, 4, 1.25 / 16))
    del GP
    out["bias_fc"] = timeit(lambda: ops.bias_dot(G2, 4, grad_scale=1.25))
    X = rnd(20, 1024, 768)
    GL = rnd(20, 1024, 768, s=1e-3)
    out["layernorm"] = timeit(lambda: ops.layernorm_dot(X, GL, 4, 1e-5, grad_scale=1.25))
    ids = torch.randint(0, 50257, (20, 1024), generator=g).to(dev)
    out["embedding_wte"] = timeit(lambda: ops.embedding_dot(ids, GL, 4, 50257))
    tab = torch.zeros(50257, 768, dtype=torch.bfloat16, device=dev)
    out["embedding_grad_tied"] = timeit(lambda: ops.embedding_train_grad(
        ids, GL, 4, 1.25, tab, accumulate=True))
    out["embedding_grad_untied"] = timeit(lambda: ops.embedding_train_grad(ids, GL, 4, 1.25,
                                                                           tab))
    del tab
    del X, GL
    A2, G2 = A[:20].contiguous(), G[:20].contiguous()
    for key, g_src in (("dot_train_grad_conv1d_c_fc", G2),
                       ("dot_train_grad_conv1d_c_attn", G2[..., :2304])):
        g_op = g_src.contiguous()
        out[key] = timeit(lambda: ops.linear_dot_train_grad(
            A2, g_op, 4, semantics=_native.SEM_PRESUM, grad_scale=1.25 / 16, bias=True,
            bias_grad_scale=1.25 / 16, conv1d=True))
        del g_op
    del A, G, A2, G2
    idp = torch.randint(0, 50257, (34, 2048), generator=g)
    idp[torch.rand(34, 2048, generator=g) < 0.9] = 50256
    idp = idp.to(dev)
    Gp = rnd(34, 2048, 768, s=1e-2)
    tab = torch.empty(50257, 768, dtype=torch.bfloat16, device=dev)
    out["embedding_grad_padded"] = timeit(lambda: ops.embedding_train_grad(idp, Gp, 2, 1.0, tab))
    del idp, Gp, tab
    A_lm = rnd(16 * 1024, 768)
    G_lm = rnd(16 * 1024, 50257, s=1e-4)
    zero = torch.zeros((), dtype=torch.bfloat16, device=dev)
    out["train_grad_lm_head_hipblaslt"] = timeit(
        lambda: torch.addmm(zero, G_lm.t(), A_lm, beta=0.0, alpha=1.25 / 16))
    del A_lm, G_lm
    Ap = rnd(10, 2048, 2048)
    Gq = rnd(10, 2048, 8192, s=1e-3)
    out["train_grad_pythia_fc"] = timeit(lambda: ops.linear_train_grad(Ap, Gq, 2, 1.25 / 8))
    At, Gt = Ap[:8].reshape(-1, 2048), Gq[:8].reshape(-1, 8192)
    out["train_grad_pythia_fc_hipblaslt"] = timeit(
        lambda: torch.addmm(zero, Gt.t(), At, beta=0.0, alpha=1.25 / 8))
    del Ap, Gq, At, Gt
    Ak = rnd(32, 1024, 1024)
    Gk = rnd(32, 1024, 4096, s=1e-3)
    Pi = rnd(16, 1024, s=0.25)
    Po = rnd(16, 4096, s=0.25)
    out["kron_fc"] = timeit(lambda: ops.kron_proj(Ak, Gk, Pi, Po, 32.0))
    del Gk
    idk = torch.randint(0, 50257, (32, 1024), generator=g).to(dev)
    PiT = rnd(50257, 16, s=0.25)
    Poe = rnd(16, 1024, s=0.25)
    out["kron_embed_wte"] = timeit(lambda: ops.kron_embed_proj(idk, Ak, PiT, Poe, 1.0))
    del Ak, idk, PiT
    src = torch.empty(1 << 29, dtype=torch.bfloat16, device=dev)
    dst = torch.empty_like(src)
    out["copy_1GiB"] = timeit(lambda: dst.copy_(src))
    out["copy_GBps"] = 2 * (1 << 30) / (out["copy_1GiB"] * 1e-3) / 1e9
    print(json.dumps(out), flush=True)


# bench op name -> kernel-leg entry at the same shape (profiles/traffic.json, from the
# FETCH_SIZE / WRITE_SIZE counter runs of `bench.py --mode kernels`)
TRAFFIC_KEYS = {"linear_valgrad[768x3072]": "valgrad_fc",
                "linear_valgrad+bias[768x3072]": "valgrad_bias_fc",
                "linear_valgrad+bias[3072x768]": "valgrad_bias_fc_out",
                "linear_valgrad+bias[768x2304]": "valgrad_bias_qkv",
                "linear_valgrad+bias[768x768]": "valgrad_bias_proj", "bias_dot": "bias_fc",
                "linear_valgrad+bias+train_grad[768x3072]": "dot_train_grad_fc",
                "linear_valgrad+bias+train_grad[3072x768]": "dot_train_grad_fc_out",
                "linear_valgrad+bias+train_grad[768x2304]": "dot_train_grad_qkv",
                "linear_valgrad+bias+train_grad[768x768]": "dot_train_grad_proj",
                "layernorm_dot": "layernorm", "embedding_dot": "embedding_wte",
                "conv1d_valgrad+bias+train_grad[768x3072]": "dot_train_grad_conv1d_c_fc",
                "conv1d_valgrad+bias+train_grad[768x2304]": "dot_train_grad_conv1d_c_attn",
                "kron_proj": "kron_fc", "kron_embed_proj": "kron_embed_wte",
                "ghost": "ghost_microbench"}


def measured_traffic(op_name):
    """HBM bytes per launch measured by the counter runs for this op's shape, or None."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    key = TRAFFIC_KEYS.get(op_name)
    if key is None or not os.path.exists(path):
        return None
    with open(path) as f:
        entry = json.load(f).get(key)
    return None if entry is None else entry.get("traffic_bytes")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--mode", choices=["full", "kernels"], default="full")
    ap.add_argument("--legs", default="gradproj,pythia,hf_gpt2",
                    help="extra legs after the GPT-2 step: gradproj, pythia, hf_gpt2 (comma "
                         "list or none)")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=60.0)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus "
              f"{args.gpus}", file=sys.stderr)
        sys.exit(2)
    assert torch.cuda.is_available(), "bench.py needs a ROCm GPU"
    dev = torch.device("cuda:0")
    from ghostsuite_amd import _native
    _native.load_library()
    if args.mode == "kernels":
        kernels_leg(dev)
        return

    import contextlib
    with contextlib.redirect_stdout(sys.stderr):
        res = gpt2_bench(args.steps, args.warmup, dev)
    log("[bench] GPT-2 step done; ghost kernel microbench")
    gk = ghost_kernel_bench(dev)
    log(f"[bench] ghost kernel T=1024: {gk['ms']:.3f} ms, {gk['tflops']:.1f} TF/s")
    sweep = ghost_sweep(dev)
    log("[bench] configs[1] T sweep done")
    emb_pad = emb_grad_pad_bench(dev)
    log(f"[bench] embedding train grad, padded batch: {emb_pad}")
    peak = achievable_peak(dev)
    log(f"[bench] achievable bf16 GEMM rate: {peak['TFLOP/s']:.0f} TFLOP/s")
    vendor = vendor_route(dev)
    log(f"[bench] fc_out outputs through hipBLASLt: {vendor['ms'] * 1e3:.1f} us")
    legs = [l for l in args.legs.split(",") if l and l != "none"]
    extra = {}
    import contextlib
    # The engines print progress like the reference does; keep stdout for the JSON line.
    with contextlib.redirect_stdout(sys.stderr):
        if "gradproj" in legs:
            extra["gradproj"] = gradproj_bench(3, 1, dev)
            log(f"[bench] gradproj: {extra['gradproj']['ms_per_step']:.1f} ms/step")
        if "pythia" in legs:
            extra["pythia"] = pythia_bench(3, 1, dev)
            log(f"[bench] pythia: {extra['pythia']['ms_per_step']:.1f} ms/step")
        if "hf_gpt2" in legs:
            extra["hf_gpt2"] = hf_gpt2_bench(5, 2, dev)
            log(f"[bench] hf_gpt2: {extra['hf_gpt2']['ms_per_step']:.1f} ms/step")

    ops = res["ops"]
    steps = args.steps
    dom_name, dom = max(ops.items(), key=lambda kv: kv[1]["ms"])
    avg_ms = dom["ms"] / dom["n"]
    achieved = dom["work"] / (avg_ms * 1e-3)
    if dom["bound"] == "mfma":
        roof = {"bound": "mfma", "kernel": dom_name, "achieved": achieved / 1e12,
                "peak": PEAK_BF16 / 1e12, "unit": "TFLOP/s", "frac": achieved / PEAK_BF16,
                "traffic": measured_traffic(dom_name), "avg_ms": avg_ms,
                "launches_per_step": dom["n"] / steps}
        roof["flops_per_launch"] = dom["work"]
        if dom.get("apart", dom["work"]) != dom["work"]:
            roof["note"] = ("flops_per_launch = the dots by the cheapest same-semantics "
                            "algorithm, 2 (n_v' + n_t) T d_in d_out, which the op executes; "
                            "its weight train gradient comes from the same GEMM and is not "
                            "counted")
            roof["if_computed_apart"] = {"flops_per_launch": dom["apart"],
                                         "rate": dom["apart"] / (avg_ms * 1e-3) / 1e12,
                                         "unit": "TFLOP/s",
                                         "note": "what the dots and the train gradient would "
                                                 "cost as two separate GEMM passes, per the "
                                                 "op's time; not a utilisation"}
    else:
        roof = {"bound": "hbm", "kernel": dom_name, "achieved": achieved / 1e9,
                "peak": PEAK_HBM / 1e9, "unit": "GB/s", "frac": achieved / PEAK_HBM,
                "traffic": measured_traffic(dom_name), "avg_ms": avg_ms,
                "launches_per_step": dom["n"] / steps}
    if roof["bound"] == "mfma":
        roof["achievable_peak"] = {**peak, "frac": roof["achieved"] / peak["TFLOP/s"],
                                   "note": "frac of the vendor library's own large-GEMM rate on "
                                           "this box; `frac` above is against the nominal "
                                           "2.5 PF/s"}
        if dom_name == "linear_valgrad+bias+train_grad[3072x768]":
            roof["vendor_route_same_outputs"] = {
                **vendor, "speedup": vendor["ms"] / avg_ms,
                "note": "the op's weight dots and weight train gradient through hipBLASLt "
                        "(isolated, no bias terms) against this op's in-step time"}
    hot_ms = sum(v["ms"] for v in ops.values()) / steps
    cpu = None if args.no_cpu_baseline else cpu_baseline(args.cpu_budget)
    value = res["n_train"] / res["t_ghost"]
    out = {
        "metric": METRIC,
        "value": value,
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": res["t_ghost"] * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (uniform token ids, random-init N(0,0.02) weights)",
        "config": {"workload": "GPT-2-small GradDotProd step, 16 train + 4 val rows, T=1024",
                   "global_batch": res["n_train"] + res["n_val"], "seq_len": res["T"],
                   "parallelism": "single GPU"},
        "plain_ms_per_step": res["t_plain"] * 1e3,
        "plain_train_rows_only_ms_per_step": res["t_plain_train"] * 1e3,
        "ms_per_step_serialised_dots": res["t_serial"] * 1e3,
        "step_overhead": res["t_ghost"] / res["t_plain"],
        "rows_per_s_total": (res["n_train"] + res["n_val"]) / res["t_ghost"],
        "hot_path_ms_per_step": hot_ms,
        "step_overhead_vs_train_rows_only": res["t_ghost"] / res["t_plain_train"],
        "step_overhead_serialised_dots": res["t_serial"] / res["t_plain"],
        "roofline": roof,
        "notes": {
            "roofline_traffic": "HBM bytes per launch from profiles/traffic.json: rocprofv3 "
                                "FETCH_SIZE / WRITE_SIZE runs of `bench.py --mode kernels` at "
                                "the same shape, scaled by the 1 GiB copy calibration; not "
                                "measured in this run",
            "tied_lm_head_dot": "not computed: the reference computes the tied lm_head's "
                                "ghost dot and then overwrites it with wte's "
                                "(supported_layers_grad_samplers_dotprod.py:130 vs :211), so "
                                "the outputs are identical without it",
        },
        "ghost_kernel": {"shape": "A[32,1024,768] G[32,1024,3072] bf16, 8 val rows first",
                         "ms": gk["ms"], "achieved": gk["tflops"], "unit": "TFLOP/s",
                         "peak": PEAK_BF16 / 1e12, "frac": gk["frac"],
                         "traffic": measured_traffic("ghost"),
                         "valgrad_same_semantics_ms": gk["valgrad_ms"],
                         "timing": {"ms_per_block": gk["block_ms"],
                                    "warmup_calls": gk["warmup_calls"],
                                    "calls_per_block": gk["calls_per_block"],
                                    "ms": "median block's average per call"},
                         "frac_of_achievable_peak": gk["tflops"] / peak["TFLOP/s"],
                         "T_sweep": sweep},
        "ops": {k: {"ms_per_step": v["ms"] / steps, "calls_per_step": v["n"] / steps,
                    "avg_us": v["ms"] / v["n"] * 1e3,
                    ("TFLOP/s" if v["bound"] == "mfma" else "GB/s"):
                        v["work"] / (v["ms"] / v["n"] * 1e-3) / (1e12 if v["bound"] == "mfma" else 1e9)}
                for k, v in sorted(ops.items(), key=lambda kv: -kv[1]["ms"])},
        "embedding_train_grad_padded_batch": emb_pad,
        "algorithms": {k: list(v) for k, v in list(res["algos"].items())[:8]},
        "cpu_baseline": cpu,
        **extra,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
