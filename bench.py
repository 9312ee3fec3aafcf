"""Benchmark of the token loop on one MI355X (BASELINE.json metric).

Default workload: a random-init Qwen3-8B-shaped model, MLX affine 4-bit
group 64 (bf16 scale/bias), bf16 KV cache; a 4096-token prompt of random ids is prefilled, then
batch-1 greedy decode. A "step" is one decode token: W untimed steps, then K timed steps issued as
the reference's pipelined loop does (step n+1 committed before step n is read back, Engine.swift:740-763),
bracketed by device synchronisation. value = decode tokens/s of the whole job (one GPU).
`--mode small` runs configs[0] instead (Qwen3-0.6B shape, 32 + 64 tokens), `--mode prefill`
configs[2] (Llama-3-8B shape, one 2048-token prefill per step), `--mode sweep` configs[3] (the
matvec / GEMM sweep), `--mode verify` the speculative verify pass (f3) on configs[1]'s model,
`--mode long` configs[4] (Qwen2.5-32B shape, 32K context, sparse decode
attention, reused prefix).

Extra objects on the JSON line:
- roofline: the dominant kernel, the persistent decode step (one launch per token: every layer,
  lm_head and the greedy token), timed with HIP events on the model's stream over its own timed
  region; achieved = algorithmic bytes per launch (every weight byte + K/V at the mean context) /
  mean launch time, against the 8 TB/s HBM peak; traffic = HBM bytes per launch from rocprofv3
  FETCH_SIZE + WRITE_SIZE (copy-kernel calibrated), read from profiles/decode_step_traffic.json
  when that file is for the same config (null otherwise), with the context it was measured at;
- step_roofline: the same accounting for the whole decode step (bytes per token at the mean context);
- prefill: prompt tokens/s of the 4096-token prefill (the config's second metric), with its flops
  (prefill_flops) against the MFMA peak;
- small_config1 / prefill_config3 / sweep_config4 / long_config5: the `--mode small`,
  `--mode prefill`, `--mode sweep` and `--mode long` results,
  each with its own roofline, measured in the same run after the decode workload;
- cpu_baseline: the CPU oracle (C restatement of the reference's semantics, all host cores) timed on
  a bounded sample: decode steps at the same context, starting from the GPU-built KV cache;
- verify_f3: the speculative verify pass (T = 2 / 5 / 8 tokens, logits of every row) on the same
  model after the decoded positions, and the tokens a pass must yield to beat plain decode steps.
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "mlx-runner_amd"), os.path.join(ROOT, "oracle")]

import configs  # noqa: E402
import mlxr  # noqa: E402

HBM_PEAK_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def model_dir(name, seed):
    base = os.environ.get("MLXR_BENCH_DIR", os.path.join(os.environ.get("TMPDIR", "/tmp"), "mlxr_bench"))
    d = os.path.join(base, f"{name}-s{seed}")
    marker = os.path.join(d, ".complete")
    if not os.path.exists(marker):
        t = time.time()
        log(f"[bench] writing synthetic {name} (seed {seed}) to {d}")
        mlxr.synth_write(configs.CONFIGS[name], seed=seed, directory=d)
        open(marker, "w").write("ok")
        log(f"[bench] synthetic model written in {time.time() - t:.1f}s")
    return d


def small_main(a):
    """the Qwen3-0.6B shape, a 32-token random prompt, then 64 greedy decode steps (the
    reference's short-context decode benchmark). The prompt and steps run once untimed, then again
    timed from a fresh prefill; value = decode tok/s over the 64 steps (two in flight, as the main
    line); roofline = the persistent step kernel (HIP events) against the HBM peak."""
    cfg = configs.CONFIGS[a.config]
    d = model_dir(a.config, a.seed)
    n_prompt, n_steps = 32, 64
    model = mlxr.Transformer(d, context_length=n_prompt + n_steps + a.step_iters + 16)
    if a.decode_mode != 1:
        model.set_decode_mode(a.decode_mode)
    greedy = mlxr.SamplingParameters.greedy()
    prompt = np.random.default_rng(a.seed).integers(0, model.vocab_size, n_prompt).astype(np.int32)

    def run():
        model.prefill(prompt, 0, greedy)
        mlxr.synchronize()
        t = time.perf_counter()
        cur = model.begin_decode_step(n_prompt, greedy)
        toks = []
        for i in range(n_steps):
            nxt = model.begin_decode_step(cur.offset + 1, greedy) if i + 1 < n_steps else None
            toks.append(model.finish(cur))
            cur = nxt
        mlxr.synchronize()
        return time.perf_counter() - t, toks

    run()
    el, toks = run()
    tok_s = n_steps / el
    mean_ctx = n_prompt + n_steps / 2
    step_ms, step_b = model.profile_kernel("step", a.step_iters, n_prompt + n_steps)
    step_gbs = step_b / (step_ms * 1e-3) / 1e9
    log(f"[bench] {a.config} decode {n_steps} steps after {n_prompt} prompt tokens: {el * 1e3:.1f} ms, {tok_s:.1f} tok/s; "
        f"step kernel {step_ms * 1e3:.1f} us, {step_gbs:.0f} GB/s")
    result = {
        "metric": "decode tok/s (bs1, 0.6B-shape 4-bit g64, 32-token prompt + 64 greedy steps) + % HBM roofline",
        "value": round(tok_s, 1), "unit": "tok/s", "n_gpus": 1, "steps": n_steps, "warmup": n_steps,
        "ms_per_step": round(el * 1e3 / n_steps, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u4 weights (affine g64, bf16 scale/bias); x as f16 hi+lo MFMA operands, fp32 accumulate, bf16 KV",
        "data": "synthetic: random-init weights N(0,0.02) from a seed, uniform random prompt ids",
        "config": {"workload": f"{a.config}: {n_prompt}-token prompt + {n_steps} greedy decode steps (configs[0])",
                   "model": a.config, "global_batch": 1, "seq_len": n_prompt + n_steps, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "kernel": "decode_step_kernel (persistent: whole token step in one launch)",
                     "achieved": round(step_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(step_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "avg_launch_us": round(step_ms * 1e3, 2), "bytes_per_launch": int(step_b)},
        "step_roofline": {"bytes_per_token": int(step_bytes(cfg, mean_ctx)),
                          "frac": round(step_bytes(cfg, mean_ctx) * tok_s / 1e9 / HBM_PEAK_GBS, 4)},
        "first_tokens": toks[:8],
    }
    model.close()
    return result


def weight_bytes(cfg):
    """Quantized bytes of every projection + lm_head (bits/8 + 4/gs bytes per weight)."""
    H, I, L, V = cfg["hidden_size"], cfg["intermediate_size"], cfg["num_hidden_layers"], cfg["vocab_size"]
    D, nH, nKV = cfg["head_dim"], cfg["num_attention_heads"], cfg["num_key_value_heads"]
    q = cfg["quantization"]
    bpw = q["bits"] / 8 + 4 / q["group_size"]
    per_layer = H * (nH + 2 * nKV) * D + nH * D * H + 3 * H * I
    return (L * per_layer + V * H) * bpw


def step_bytes(cfg, ctx):
    """Algorithmic HBM bytes of one decode token at context ctx (SURVEY 8d accounting): weights,
    the bf16 K/V read (2 * nKV * D * ctx * 2 bytes per layer), the KV append, the embedding row and
    the logits write+read."""
    L, D, nKV, V, H = cfg["num_hidden_layers"], cfg["head_dim"], cfg["num_key_value_heads"], cfg["vocab_size"], cfg["hidden_size"]
    q = cfg["quantization"]
    kv = L * 2 * nKV * D * ctx * 2 + L * 2 * nKV * D * 2
    return weight_bytes(cfg) + kv + H * (q["bits"] / 8 + 4 / q["group_size"]) + V * 4 * 2


MFMA_PEAK_TFS = 2500.0   # MI355X dense bf16 / f16


def prefill_flops(cfg, T, pos0=0):
    """Algorithmic flops of a T-token prefill chunk at position pos0: every projection (2 flops per
    weight per token), causal attention (q.k and p.v: 4 * head_dim flops per query, key, head) and the
    lm_head for the last token."""
    H, I, L, V = cfg["hidden_size"], cfg["intermediate_size"], cfg["num_hidden_layers"], cfg["vocab_size"]
    D, nH, nKV = cfg["head_dim"], cfg["num_attention_heads"], cfg["num_key_value_heads"]
    per_layer = H * (nH + 2 * nKV) * D + nH * D * H + 3 * H * I
    keys = T * pos0 + T * (T + 1) // 2
    return L * (2 * T * per_layer + 4 * D * nH * keys) + 2 * H * V


def prefill_main(a):
    """one sequence of random ids through the prefill (quantized GEMMs + causal flash
    attention); value = prompt tok/s, roofline = the whole prefill's flops against the MFMA peak."""
    cfg = configs.CONFIGS[a.config]
    d = model_dir(a.config, a.seed)
    model = mlxr.Transformer(d, context_length=a.context + 64)
    greedy = mlxr.SamplingParameters.greedy()
    prompt = np.random.default_rng(a.seed).integers(0, model.vocab_size, a.context).astype(np.int32)
    for _ in range(max(1, a.warmup)):
        model.prefill(prompt, 0, greedy)
    mlxr.synchronize()
    times = []
    for _ in range(max(1, a.steps)):
        t = time.perf_counter()
        model.prefill(prompt, 0, greedy)
        mlxr.synchronize()
        times.append(time.perf_counter() - t)
    el = sum(times) / len(times)
    fl = prefill_flops(cfg, a.context)
    tfs = fl / el / 1e12
    log(f"[bench] prefill {a.context} tokens: {el * 1e3:.1f} ms ({a.context / el:.0f} tok/s, {tfs:.0f} TFLOP/s)")
    result = {
        "metric": "prefill tok/s (2048-token prompt, 8B-shape 4-bit g64) + % MFMA peak",
        "value": round(a.context / el, 1), "unit": "tok/s", "n_gpus": 1, "steps": len(times), "warmup": max(1, a.warmup),
        "ms_per_step": round(el * 1e3, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u4 weights (affine g64, bf16 scale/bias); f16 GEMM operands, bf16 hi/lo attention, fp32 accumulate",
        "data": "synthetic: random-init weights N(0,0.02) from a seed, uniform random prompt ids",
        "config": {"workload": f"{a.config}: one {a.context}-token prefill (configs[2])", "model": a.config,
                   "global_batch": 1, "seq_len": a.context, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "mfma", "kernel": "whole prefill (tile GEMMs, flash attention, norms)",
                     "achieved": round(tfs, 1), "peak": MFMA_PEAK_TFS, "unit": "TFLOP/s",
                     "frac": round(tfs / MFMA_PEAK_TFS, 4), "traffic": None, "flops": int(fl)},
    }
    model.close()
    return result


def sweep_main(a):
    """the quantized matvec / GEMM sweep on 8B-shape projections. Weights are random code
    words with random bf16 scales / biases (every bit pattern is a valid code stream at any width;
    parity is the kernel tests' job), activations N(0, 1) rounded to bf16 values (stored fp32). T = 1: the decode matvec (mlxr_k_qmv),
    T = 4: the small-batch kernel (mlxr_k_qmm), T = 512: the prefill GEMM (mlxr_k_qgemm). HIP events
    around `iters` back-to-back calls; bytes = N*K*(b/8 + 4/gs) + T*K*4 + T*N*4, flops = 2*T*N*K."""
    rng = np.random.default_rng(a.seed)
    shapes = [(4096, 14336), (14336, 4096), (4096, 151936)]
    quants = [(3, 32), (4, 64), (6, 128), (8, 64)]
    cells = []
    for K, N in shapes:
        for bits, gs in quants:
            w = mlxr.DeviceArray.from_numpy(rng.integers(0, 2**32, (N, K * bits // 32), dtype=np.uint32))
            sc = mlxr.DeviceArray.from_numpy((rng.uniform(0.001, 0.05, (N, K // gs)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16))
            bi = mlxr.DeviceArray.from_numpy((rng.uniform(-0.2, 0.2, (N, K // gs)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16))
            qm = (mlxr.QMat * 1)(mlxr.QMat(w.ptr, sc.ptr, bi.ptr, None, N))
            for T in (1, 4, 512):
                xv = rng.normal(0, 1, (T, K)).astype(np.float32)
                xv = ((xv.view(np.uint32) + 0x7FFF + ((xv.view(np.uint32) >> 16) & 1)) & 0xFFFF0000).view(np.float32)   # bf16 values
                x = mlxr.DeviceArray.from_numpy(xv)
                y = mlxr.DeviceArray.zeros((T, N), np.float32)
                if T == 1:
                    call = lambda: mlxr.lib.mlxr_k_qmv(qm, 1, K, bits, gs, 0, x.ptr, None, 0.0, y.ptr, 0)
                elif T == 4:
                    call = lambda: mlxr.lib.mlxr_k_qmm(qm, 1, K, bits, gs, 0, T, x.ptr, K, y.ptr, N)
                else:
                    call = lambda: mlxr.lib.mlxr_k_qgemm(qm, K, bits, gs, 0, T, x.ptr, K, y.ptr, N)
                mlxr.check(call())
                mlxr.synchronize()
                iters = 20 if T == 512 else 50
                mlxr.check(mlxr.lib.mlxr_timer_start())
                for _ in range(iters):
                    mlxr.check(call())
                ms = ctypes.c_float()
                mlxr.check(mlxr.lib.mlxr_timer_stop(ms))
                us = ms.value * 1e3 / iters
                byt = N * K * (bits / 8 + 4 / gs) + T * K * 4 + T * N * 4
                cell = {"K": K, "N": N, "bits": bits, "gs": gs, "T": T, "us": round(us, 2),
                        "GBs": round(byt / us / 1e3, 1), "TFLOPs": round(2 * T * N * K / us / 1e6, 2)}
                cells.append(cell)
                log(f"[bench] sweep K={K} N={N} {bits}b g{gs} T={T}: {us:8.1f} us  {cell['GBs']:7.0f} GB/s  {cell['TFLOPs']:6.1f} TFLOP/s")
                x.free(); y.free()
            w.free(); sc.free(); bi.free()
    dec = [c for c in cells if c["T"] == 1]
    gemm = [c for c in cells if c["T"] == 512]
    best_dec = max(dec, key=lambda c: c["GBs"])
    result = {
        "metric": "quantized matvec / GEMM sweep (8B-shape projections, configs[3])",
        "value": round(sum(c["GBs"] for c in dec) / len(dec), 1), "unit": "GB/s (mean over the T = 1 cells)",
        "n_gpus": 1, "steps": len(cells), "warmup": 1, "ms_per_step": None, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "u3/u4/u6/u8 weights (bf16 scale/bias); fp32 activations; T = 1: fp32 arithmetic; T = 4 and exact codes and x as f16 hi + lo on the f16 matrix cores (the lo products skipped where x is bf16-valued, as here), group scale / bias in fp32, fp32 accumulate",
        "data": "synthetic: random code words and bf16 scales / biases, N(0,1) activations rounded to bf16",
        "config": {"workload": "configs[3]: K,N in (4096,14336),(14336,4096),(4096,151936) x 3b g32, 4b g64, 6b g128, 8b g64 x T in 1,4,512"},
        "roofline": {"bound": "hbm", "kernel": f"qmv_kernel, best cell K={best_dec['K']} N={best_dec['N']} {best_dec['bits']}b",
                     "achieved": best_dec["GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(best_dec["GBs"] / HBM_PEAK_GBS, 4), "traffic": None},
        "gemm_T512": {"best_TFLOPs": max(c["TFLOPs"] for c in gemm), "peak": MFMA_PEAK_TFS},
        "cells": cells,
    }
    return result


def verify_main(a):
    """f3 alone: the speculative verify pass on configs[1]'s model after a `context`-token prefill
    (T = 2 / 5 / 8 tokens, logits of every row; 3 warm-up + `steps` timed passes each)."""
    d = model_dir(a.config, a.seed)
    model = mlxr.Transformer(d, context_length=a.context + 16)
    greedy = mlxr.SamplingParameters.greedy()
    prompt = np.random.default_rng(a.seed).integers(0, model.vocab_size, a.context).astype(np.int32)
    model.prefill(prompt, 0, greedy)
    mlxr.synchronize()
    ms = {}
    for T in (2, 5, 8):
        for _ in range(3):
            model.forward(prompt[:T], a.context, all_logits=True)
        mlxr.synchronize()
        t = time.perf_counter()
        for _ in range(a.steps):
            model.forward(prompt[:T], a.context, all_logits=True)
        mlxr.synchronize()
        ms[T] = (time.perf_counter() - t) / a.steps * 1e3
        log(f"[bench] verify T={T}: {ms[T]:.2f} ms")
    model.close()
    return {"metric": "speculative verify pass ms (T tokens, all logits)", "value": round(ms[5], 3), "unit": "ms",
            "higher_is_better": False, "steps": a.steps,
            "config": {"workload": f"{a.config}: T-token verify pass at context {a.context} (f3)"},
            "T": list(ms), "ms": [round(v, 3) for v in ms.values()]}


def long_main(a):
    """Qwen2.5-32B shape, 32768-token context with sparse decode attention. Turn 1
    prefills the first 30000 ids; turn 2 reuses that prefix (reusable_prefix), prefills the remaining
    ids and decodes `steps` greedy tokens (two in flight)."""
    cfg = configs.CONFIGS[a.config]
    d = model_dir(a.config, a.seed)
    model = mlxr.Transformer(d, context_length=a.context, sparse=mlxr.SparseAttention(min_context=5128))
    if a.no_graphs:
        model.set_graphs(False)
    total = model.max_seq - a.steps - a.warmup - 8      # the prompt leaves room for the decoded tokens
    first_turn = min(30000, total - 8)
    greedy = mlxr.SamplingParameters.greedy()
    ids = np.random.default_rng(a.seed).integers(0, model.vocab_size, total).astype(np.int32)
    t = time.perf_counter()
    model.prefill(ids[:first_turn], 0, greedy)
    mlxr.synchronize()
    t1 = time.perf_counter() - t
    reuse = model.reusable_prefix(first_turn, first_turn)
    t = time.perf_counter()
    tok = model.prefill(ids[reuse:], reuse, greedy)
    mlxr.synchronize()
    t2 = time.perf_counter() - t
    log(f"[bench] turn 1 prefill {first_turn} tokens: {t1:.2f} s; turn 2 reuses {reuse}, prefills {total - reuse} in {t2 * 1e3:.0f} ms")
    pos = total

    def run(n, pos, first):
        toks = []
        cur = model.begin_decode_step(pos, greedy)
        for i in range(n):
            nxt = model.begin_decode_step(cur.offset + 1, greedy) if i + 1 < n else None
            toks.append(model.finish(cur))
            cur = nxt
        return toks

    run(a.warmup, pos, tok)
    pos += a.warmup
    mlxr.synchronize()
    t = time.perf_counter()
    toks = run(a.steps, pos, tok)
    mlxr.synchronize()
    el = time.perf_counter() - t
    tok_s = a.steps / el
    # sparse accounting: weights + per layer the index scan and the attended keys
    L, nKV, D = cfg["num_hidden_layers"], cfg["num_key_value_heads"], cfg["head_dim"]
    ctx = pos + a.steps // 2
    blocks = (ctx - 512) // 4
    attended = 4 + 4 * min(512, blocks) + 512
    sb = weight_bytes(cfg) + L * (blocks * nKV * D * 2 + attended * nKV * D * 2 * 2)
    log(f"[bench] long-context decode {a.steps} steps: {el * 1e3:.1f} ms, {tok_s:.1f} tok/s ({sb * tok_s / 1e9:.0f} GB/s algorithmic)")
    result = {
        "metric": "decode tok/s (bs1, 32B-shape 4-bit g64, 32K context, sparse attention) + % HBM roofline",
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(el * 1e3 / a.steps, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u4 weights (affine g64, bf16 scale/bias); x as f16 hi+lo MFMA operands (fp32-level), fp32 accumulate, bf16 KV",
        "data": "synthetic: random-init weights N(0,0.02) from a seed, uniform random ids",
        "config": {"workload": f"{a.config}: {total}-token context, {reuse}-token reused prefix, sparse decode (configs[4])",
                   "model": a.config, "global_batch": 1, "seq_len": total + a.warmup + a.steps, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "kernel": "whole decode step (kernel-per-op graph; sparse attention)",
                     "achieved": round(sb * tok_s / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(sb * tok_s / 1e9 / HBM_PEAK_GBS, 4), "traffic": None, "bytes_per_token": int(sb)},
        "prefill": {"turn1_tokens": first_turn, "turn1_s": round(t1, 3), "reused": reuse, "turn2_tokens": total - reuse,
                    "turn2_ms": round(t2 * 1e3, 1)},
        "first_tokens": toks[:8],
    }
    model.close()
    return result


def cpu_baseline(d, model, cfg, ctx, tokens, budget_s):
    import oracle
    t0 = time.time()
    ref = oracle.Model(d, model.max_seq)
    L, nKV, D = cfg["num_hidden_layers"], cfg["num_key_value_heads"], cfg["head_dim"]
    for layer in range(L):
        k, v = model.read_kv(layer, ctx, nKV, D)
        ref.set_kv(layer, k, v)
    log(f"[bench] oracle loaded with the GPU's KV cache in {time.time() - t0:.1f}s")
    done, t = 0, time.time()
    pos = ctx
    while done < tokens:
        ref.forward(np.array([7 + done], np.int32), pos)
        pos += 1
        done += 1
        if time.time() - t > budget_s:
            break
    el = time.time() - t
    ref.close()
    return {"value": done / el, "unit": "tok/s", "cores": oracle.threads(), "kind": "port",
            "sample": f"{done} greedy decode token(s) of the same model at context {ctx} (KV cache copied from the GPU run), "
                      f"fp32 C oracle, OpenMP over {oracle.threads()} host threads; {el:.1f}s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--config", default="qwen3-8b", choices=sorted(configs.CONFIGS))
    ap.add_argument("--context", type=int, default=4096, help="prefilled prompt tokens")
    ap.add_argument("--seed", type=int, default=2)
    ap.add_argument("--cpu-tokens", type=int, default=2)
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="decode only: skip the small_config1, prefill_config3, sweep_config4 and long_config5 "
                         "sub-objects (configs[0], [2], [3] and [4])")
    ap.add_argument("--kernel-iters", type=int, default=360)
    ap.add_argument("--step-iters", type=int, default=64)
    ap.add_argument("--no-graphs", action="store_true",
                    help="launch the kernel-per-op decode step kernel by kernel (profiling) instead of as a hipGraph")
    ap.add_argument("--decode-mode", type=int, default=1, choices=[0, 1, 2],
                    help="1: persistent decode step, 0: kernel per op (repacked tiles), 2: kernel per op (MLX layout)")
    ap.add_argument("--mode", default="decode", choices=["decode", "small", "prefill", "sweep", "long", "verify"],
                    help="decode: configs[1] (default); small: configs[0] (qwen3-0.6b, 32 + 64 tokens); prefill: "
                         "configs[2] (llama3-8b, 2048 tokens unless given); sweep: configs[3]; long: configs[4] "
                         "(qwen2.5-32b, 32768-token context, sparse)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MB",
                    help="only run 3 device-to-device copy kernels of MB MiB each (calibrates rocprofv3 byte counters)")
    a = ap.parse_args()
    if a.copy_probe:
        import torch
        src = torch.empty(a.copy_probe << 18, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": a.copy_probe << 20, "launches": 3}))
        return
    if a.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU: multi-GPU runs are not part of it (see DESIGN.md, sharding)",
                          "n_gpus": a.gpus}))
        sys.exit(2)
    if mlxr.device_count() < 1:
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    if a.mode == "prefill":
        if "--config" not in sys.argv:
            a.config = "llama3-8b"
        if "--context" not in sys.argv:
            a.context = 2048
        if "--steps" not in sys.argv:
            a.steps = 5
        if "--warmup" not in sys.argv:
            a.warmup = 1
        print(json.dumps(prefill_main(a)), flush=True)
        return
    if a.mode == "sweep":
        print(json.dumps(sweep_main(a)), flush=True)
        return
    if a.mode == "verify":
        print(json.dumps(verify_main(a)), flush=True)
        return
    if a.mode == "small":
        if "--config" not in sys.argv:
            a.config = "qwen3-0.6b"
        print(json.dumps(small_main(a)), flush=True)
        return
    if a.mode == "long":
        if "--config" not in sys.argv:
            a.config = "qwen2.5-32b"
        if "--context" not in sys.argv:
            a.context = 32768
        if "--steps" not in sys.argv:
            a.steps = 128
        if "--warmup" not in sys.argv:
            a.warmup = 4
        print(json.dumps(long_main(a)), flush=True)
        return
    cfg = configs.CONFIGS[a.config]
    d = model_dir(a.config, a.seed)
    need = a.context + a.warmup + a.steps + a.step_iters + 16
    t = time.time()
    model = mlxr.Transformer(d, context_length=need)
    log(f"[bench] model loaded in {time.time() - t:.1f}s ({model.weight_bytes / 1e9:.2f} GB of weights, {model.quant_description})")
    model.set_decode_mode(a.decode_mode)
    if a.no_graphs:
        model.set_graphs(False)
    greedy = mlxr.SamplingParameters.greedy()
    prompt = np.random.default_rng(a.seed).integers(0, model.vocab_size, a.context).astype(np.int32)

    # prefill (timed separately; warm the kernels once on a short prompt first)
    model.prefill(prompt[:64], 0, greedy)
    mlxr.synchronize()
    t = time.perf_counter()
    first = model.prefill(prompt, 0, greedy)
    mlxr.synchronize()
    prefill_s = time.perf_counter() - t
    log(f"[bench] prefill {a.context} tokens: {prefill_s * 1e3:.1f} ms ({a.context / prefill_s:.0f} tok/s)")

    # decode: warmup, then K timed steps, two in flight
    pos = a.context

    def run(n, pos):
        toks = []
        cur = model.begin_decode_step(pos, greedy)
        for i in range(n):
            nxt = model.begin_decode_step(cur.offset + 1, greedy) if i + 1 < n else None
            toks.append(model.finish(cur))
            cur = nxt
        return toks

    run(a.warmup, pos)
    pos += a.warmup
    mlxr.synchronize()
    t = time.perf_counter()
    toks = run(a.steps, pos)
    mlxr.synchronize()
    el = time.perf_counter() - t
    tok_s = a.steps / el
    mean_ctx = pos + a.steps / 2
    sb = step_bytes(cfg, mean_ctx)
    log(f"[bench] decode {a.steps} steps: {el * 1e3:.1f} ms, {tok_s:.1f} tok/s, {sb * tok_s / 1e9:.0f} GB/s algorithmic")

    # dominant kernel: the persistent decode step, HIP events on the model stream (the context runs on
    # from the last decoded position; steps overwrite the history after it)
    step_ms, step_b = model.profile_kernel("step", a.step_iters, pos + a.steps)
    step_gbs = step_b / (step_ms * 1e-3) / 1e9
    log(f"[bench] kernel step   : {step_ms * 1e3:8.1f} us  {step_b / 1e6:8.2f} MB  {step_gbs:7.0f} GB/s")
    traffic, traffic_ctx = None, None
    tf = os.path.join(ROOT, "profiles", "decode_step_traffic.json")
    if os.path.exists(tf):
        with open(tf) as f:
            t = json.load(f)
        if t.get("config") == a.config:   # measured at the context it names (K/V is ~12% of the bytes)
            traffic = int(t["bytes_per_launch"])
            traffic_ctx = t.get("context")
    # the kernel-per-op path's decode kernels (the graph fallback), for reference
    kern = {}
    for kind in ("gateup", "down", "qkv", "o", "head", "attn"):
        iters = a.kernel_iters if kind != "head" else 20
        ms, b = model.profile_kernel(kind, iters, int(mean_ctx))
        kern[kind] = {"ms": ms, "bytes": b, "GBs": b / (ms * 1e-3) / 1e9}
        log(f"[bench] kernel {kind:7s}: {ms * 1e3:8.1f} us  {b / 1e6:8.2f} MB  {kern[kind]['GBs']:7.0f} GB/s")

    result = {
        "metric": "decode tok/s (bs1, 8B-shape 4-bit g64) + % HBM roofline; prefill tok/s",
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(el * 1e3 / a.steps, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u4 weights (affine g64, bf16 scale/bias); x as f16 hi+lo MFMA operands (fp32-level, 1e-3 gate), "
                 "fp32 accumulate, bf16 KV",
        "data": "synthetic: random-init weights N(0,0.02) from a seed, uniform random prompt ids",
        "config": {"workload": f"{a.config}: {a.context}-token prefilled context + greedy decode (configs[1])",
                   "model": a.config, "global_batch": 1, "seq_len": a.context + a.warmup + a.steps, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "kernel": "decode_step_kernel (persistent: whole token step in one launch)",
                     "achieved": round(step_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(step_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "avg_launch_us": round(step_ms * 1e3, 2), "bytes_per_launch": int(step_b),
                     "context": pos + a.steps, "traffic_context": traffic_ctx},
        "step_roofline": {"achieved": round(sb * tok_s / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(sb * tok_s / 1e9 / HBM_PEAK_GBS, 4), "bytes_per_token": int(sb),
                          "tok_s_at_100pct": round(HBM_PEAK_GBS * 1e9 / sb, 1)},
        "prefill": {"tokens": a.context, "tok_s": round(a.context / prefill_s, 1), "ms": round(prefill_s * 1e3, 1),
                    "tflops": round(prefill_flops(cfg, a.context) / prefill_s / 1e12, 1),
                    "mfma_frac": round(prefill_flops(cfg, a.context) / prefill_s / 1e12 / MFMA_PEAK_TFS, 4)},
        "kernels_us": {k: round(v["ms"] * 1e3, 2) for k, v in kern.items()},
        "first_tokens": [first] + toks[:8],
    }
    if not a.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(d, model, cfg, pos + a.steps, a.cpu_tokens, a.cpu_budget)
    # speculative verify (f3): one T-token pass with the logits of every row, after the decoded
    # positions (their K/V rows are scratch past the measured context)
    ver = {}
    for T in (2, 5, 8):
        vt = prompt[:T]
        for _ in range(3):
            model.forward(vt, pos + a.steps, all_logits=True)
        mlxr.synchronize()
        t = time.perf_counter()
        for _ in range(10):
            model.forward(vt, pos + a.steps, all_logits=True)
        mlxr.synchronize()
        ver[T] = (time.perf_counter() - t) / 10 * 1e3
        log(f"[bench] verify T={T}: {ver[T]:.2f} ms")
    step_ms_mean = el * 1e3 / a.steps
    result["verify_f3"] = {
        "workload": f"{a.config}: T-token batched pass (all logits) at context {pos + a.steps}, eager launches",
        "T": list(ver), "ms": [round(v, 3) for v in ver.values()], "decode_step_ms": round(step_ms_mean, 4),
        # a verify pass yields its accepted drafts plus one token: it pays from this many tokens per pass
        "tokens_per_pass_to_break_even": {str(T): round(v / step_ms_mean, 2) for T, v in ver.items()}}
    model.close()
    if not a.no_extra:
        # the other workloads, measured in the same run (short: seconds of GPU time each)
        sa = argparse.Namespace(**vars(a))
        sa.config, sa.step_iters = "qwen3-0.6b", 64
        result["small_config1"] = _sub(small_main(sa))
        pa = argparse.Namespace(**vars(a))
        pa.config, pa.context, pa.steps, pa.warmup = "llama3-8b", 2048, 5, 1
        result["prefill_config3"] = _sub(prefill_main(pa))
        result["sweep_config4"] = _sub(sweep_main(argparse.Namespace(**vars(a))))
        la = argparse.Namespace(**vars(a))
        la.config, la.context, la.steps, la.warmup = "qwen2.5-32b", 32768, 64, 4
        result["long_config5"] = _sub(long_main(la))
    print(json.dumps(result), flush=True)


def _sub(r):
    """A workload's result as a sub-object of the main line (without the fields the line already has)."""
    return {k: v for k, v in r.items() if k not in ("n_gpus", "higher_is_better", "scaling", "vs_baseline", "data")}


if __name__ == "__main__":
    main()
