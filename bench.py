#!/usr/bin/env python3
"""Batch-1 greedy decode of the Qwen2.5-7B-shaped Q4_K_M model on one MI355X.

Workload (benchmark config 5): a synthetic Qwen2.5-7B-shaped model (hidden
3584, 28 layers, 28 Q / 4 KV heads, head_dim 128, FFN 18944, vocab 152064,
untied LM head, rope_theta 1e6), random-init N(0, 0.02) weights quantized
with the reference's q4km recipe (Q4_K q/k/o/gate/up, Q8_0 v/embeddings/LM
head, Q6_K ffn_down), generated in HBM.  The protocol is llama-bench's
(src/bin/llama-bench.rs:113-141): an untimed benchmark_tokens of 8 prompt
tokens and 1 decode step (plus one untimed round with `--warmup` decode
steps), then `--rounds` timed rounds of benchmark_tokens (src/engine.rs:
189-223: reset, prefill the 512-token random prompt with the batched MFMA
path, then `--steps` greedy decode steps, each one token through the whole
model, replayed from a captured hipGraph with the token and position kept on
the device), and the round that is the median by prefill + decode time.

Prints ONE JSON line: that round's decode tok/s as `value` (and llama-bench's
keys under "llama_bench"), the whole-step HBM rate, the dominant kernel's
roofline (HIP-event timing of its own launches) and the CPU baseline (the
oracle's restated AVX2 path on this host's cores, at the GPU's decode
positions, on a bounded sample of the same model).  `--workload cfg3|cfg4` runs the 0.5B and
1.5B end-to-end configs the same way; `--gemv` runs configs 1 and 2;
`--load` times the SafeTensors loader's load-time quantization.
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import pathlib
import sys
import time

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent
PEAK_HBM_GBS = 8000.0
PEAK_F16_FLOPS = 2.5e15  # dense f16 MFMA
METRIC = "batch-1 decode tok/s + achieved HBM GB/s (% of peak), Qwen2.5-7B-shape Q4_K_M"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def package():
    pkg = ROOT / "llama.rs_amd"
    spec = importlib.util.spec_from_file_location(
        "llama_rs_amd", pkg / "__init__.py", submodule_search_locations=[str(pkg)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["llama_rs_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def host_threads() -> int:
    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return n


def prefill_flops(cfg, n: int) -> float:
    """Algorithmic FLOPs of an n-token prefill from position 0: 2 per weight per
    token for every layer matrix, the LM head on the last token only, and the
    causal attention products (q.k and p.v, 2 FLOPs per multiply-add)."""
    H, F, KV, L = cfg.hidden_size, cfg.intermediate_size, cfg.kv_width, cfg.num_hidden_layers
    per_layer = H * H + 2 * KV * H + H * H + 3 * F * H
    linear = 2.0 * n * L * per_layer + 2.0 * cfg.vocab_size * H
    attn = 2.0 * 2 * L * cfg.num_attention_heads * cfg.head_dim * (n * (n + 1) / 2)
    return linear + attn


def kv_bytes_per_token(cfg, pos: int) -> int:
    """K and V of positions 0..pos read once per KV head, plus the new row written."""
    row = cfg.kv_width * 4
    return cfg.num_hidden_layers * 2 * ((pos + 1) * row + row)


def cpu_baseline(llrs, model, kv, prompt_len: int, first_token: int, seconds: float, label: str) -> dict:
    """The oracle's restated AVX2 path (src/simd.rs, the reference's default
    backend) timed on this host's cores at the positions the GPU decodes: its
    state is seeded with the GPU cache's K/V rows of the prompt (the GPU's
    prefill), then it decodes greedily from position `prompt_len` with
    `first_token`, each step attending over every earlier position as the
    GPU's does.  Three samples: all host threads (the reference's default,
    src/backend.rs:99-106), one thread, and the scalar path (the parity
    oracle) on all threads, each for about `seconds` (one third for the
    scalar one)."""
    sys.path.insert(0, str(ROOT / "tests"))
    from oracle_ffi import AVX2, SCALAR, Oracle

    threads = host_threads()
    mc = model.config()
    shm = pathlib.Path("/dev/shm") if os.path.isdir("/dev/shm") else pathlib.Path("/tmp")
    path = shm / f"llrs_bench_{os.getpid()}.gguf"
    rows = {(l, w): kv.layer(l, w, prompt_len) for l in range(mc.num_hidden_layers) for w in ("k", "v")}
    out = {}
    try:
        t0 = time.perf_counter()
        model.export_gguf(path)
        log(f"cpu: exported model to {path} in {time.perf_counter() - t0:.1f}s")
        for name, kernel, th, budget in (("all", AVX2, threads, seconds), ("one", AVX2, 1, seconds),
                                         ("scalar", SCALAR, threads, seconds / 3)):
            om = Oracle().load(path, kernel=kernel, threads=th)
            om.new_state(prompt_len + 130)
            for (l, w), r in rows.items():
                om.load_kv(l, w, r)
            tok, n, t0 = first_token, 0, time.perf_counter()
            while n < 128 and (n < 2 or time.perf_counter() - t0 < budget):
                om.forward_token(tok, prompt_len + n, True)
                tok = om.argmax()
                n += 1
            dt = time.perf_counter() - t0
            out[name] = (n, dt, th)
            log(f"cpu {name}: {n} steps at positions {prompt_len}-{prompt_len + n - 1} on {th} "
                f"threads: {n / dt:.3f} tok/s")
            del om
    finally:
        if path.exists():
            path.unlink()
    n, dt, th = out["all"]
    n1, dt1, _ = out["one"]
    ns, dts, _ = out["scalar"]
    return {"value": round(n / dt, 4), "unit": "tok/s", "cores": th, "kind": "port",
            "sample": f"{n} greedy decode steps at positions {prompt_len}-{prompt_len + n - 1} (the "
                      f"GPU's decode positions) of the same {label} model, the oracle seeded with the "
                      f"GPU's K/V rows of the {prompt_len}-token prompt; the oracle's restated AVX2 "
                      f"path (src/simd.rs) with the reference's row-parallel policy on {th} threads; "
                      f"the Rust reference itself cannot be built here",
            "one_thread": {"value": round(n1 / dt1, 4), "cores": 1,
                           "sample": f"{n1} steps from position {prompt_len}, AVX2 path"},
            "scalar": {"value": round(ns / dts, 4), "cores": th,
                       "sample": f"{ns} steps from position {prompt_len}, scalar path (the parity oracle)"}}


COPY_BYTES = 256 << 20  # calibration copy: 256 MiB, 4 times


def projection_only(llrs, be, model, which: str, iters: int) -> int:
    """One projection's launches (every layer, `iters` times) plus a known-size
    device copy, so that rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of the GEMV
    kernel can be scaled by what the same counter reads for the copy."""
    if which == "layers":
        # The persistent kernel at a decode-like position (520 cached rows).
        kv = llrs.KVCache(model, 1024)
        model.prefill(np.arange(520, dtype=np.uint32) * 7 % model.config().vocab_size, 0, kv)
        us, nb = model.profile_layers(kv, iters)
    else:
        kv = llrs.KVCache(model, 64)
        us, nb = model.profile_projection(kv, which, iters)
    lib = llrs.lib()
    import ctypes as C
    src, dst = C.c_void_p(), C.c_void_p()
    llrs._check(lib.llrs_device_alloc(be.handle, COPY_BYTES, C.byref(src)))
    llrs._check(lib.llrs_device_alloc(be.handle, COPY_BYTES, C.byref(dst)))
    try:
        for _ in range(4):
            llrs._check(lib.llrs_device_copy(be.handle, dst, src, COPY_BYTES))
    finally:
        lib.llrs_device_free(be.handle, src)
        lib.llrs_device_free(be.handle, dst)
    print(json.dumps({"projection": which, "avg_us": round(us, 2), "bytes": nb,
                      "copy_bytes": COPY_BYTES, "copies": 4}), flush=True)
    return 0


# Types the tuned digit GEMV takes; F32/F16/BF16 run the vectorized float
# GEMV (16-byte loads, rows sharing x), ragged shapes the wave-per-row one.
TUNED_TYPES = ("Q4K", "Q5K", "Q6K", "Q8_0", "Q5_0", "Q4_0", "Q4_1", "Q5_1")
FLOAT_TYPES = ("F32", "F16", "BF16")


LDS_PROBE_MODES = ("read32 conflict-free", "read64 conflict-free", "read128 conflict-free",
                   "read32 one bank", "write128 conflict-free", "read128 MFMA fragment, 144-byte rows",
                   "read128 MFMA fragment, 176-byte rows", "write128 staging, 144-byte rows",
                   "read128 256 B runs, unaligned", "read128 256 B runs, aligned",
                   "write128 chunk-major staging, swizzled", "write128 chunk-major staging, plain")


def lds_probe(llrs, be, iters: int, reps: int = 1) -> int:
    """The LDS access-pattern probe (llrs_debug_lds_probe): each mode `reps`
    times, 512 workgroups of 256 threads, `iters` LDS accesses per thread; run
    under rocprofv3 --pmc SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE to read what
    the counters report for known bank patterns.  With iters 1 the kernels do
    almost nothing: under rocprofv3 --kernel-trace their durations are the
    floor of a launch."""
    lib = llrs.lib()
    out = []
    for mode, name in enumerate(LDS_PROBE_MODES):
        t0 = time.perf_counter()
        for _ in range(reps):
            llrs._check(lib.llrs_debug_lds_probe(be.handle, mode, 512, iters))
        dt = (time.perf_counter() - t0) / reps
        out.append({"mode": mode, "pattern": name, "blocks": 512, "iters": iters, "reps": reps,
                    "ms": round(dt * 1e3, 3)})
        log(f"lds probe mode {mode} ({name}): {dt * 1e3:.2f} ms")
    print(json.dumps({"lds_probe": out}), flush=True)
    return 0


def gemv_cpu(oracle, kernel, threads: int, data: bytes, ty: int, rows: int, cols: int,
             x: np.ndarray, reps: int) -> float:
    """Median seconds of `reps` oracle matvecs (CpuBackend::matvec with the
    reference's row-parallel policy, src/backend.rs:143-162), after one
    untimed call."""
    buf = np.frombuffer(data, dtype=np.uint8)
    y = np.empty(rows, np.float32)
    import ctypes as C
    F32P = C.POINTER(C.c_float)
    call = lambda: oracle.lib.oq_matvec(buf.ctypes.data, ty, rows, cols, x.ctypes.data_as(F32P),
                                        y.ctypes.data_as(F32P), kernel, threads, 128 * 1024)
    assert call() == 0
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        call()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts))


def gemv_sweep(llrs, be, cpu_reps: int) -> int:
    """Configs 1 and 2: single batch-1 GEMVs through KernelBackend::matvec
    (llrs_matvec_dev on device buffers).  Config 1: Q4_K 8960 x 1536 (seed 1);
    config 2: every type at 18944 x 3584 and 3584 x 18944 (seed 2).  Each
    tensor is uploaded as many times as makes >= 1.2 GB, and the launches
    rotate over the copies, so the 256 MB MALL cannot serve a repeat; the
    timed loop is one synchronisation around n launches.  Algorithmic bytes
    = weights + x + y.

    With cpu_reps > 0 every case is also timed on the host through the
    oracle's restatement of CpuBackend::matvec (the reference cannot be built
    here): its AVX2 dots (src/simd.rs; types without one use the scalar dot,
    as the reference does) on all host threads and on one, and its scalar
    dots on all threads, each the median of cpu_reps calls."""
    import ctypes as C
    QT = llrs.QuantType
    lib = llrs.lib()
    oracle = None
    if cpu_reps > 0:
        sys.path.insert(0, str(ROOT / "tests"))
        from oracle_ffi import AVX2, SCALAR, Oracle
        oracle = Oracle()
        threads = host_threads()
    cases = [("cfg1", QT.Q4K, 8960, 1536, 1)]
    # The fixed cost of a launch: 64 rows (32 workgroups), a few hundred KB.
    cases += [("floor", QT.Q4K, 64, 3584, 2), ("floor", QT.Q4K, 64, 18944, 2)]
    for name in ("Q4_0", "Q4_1", "Q5_0", "Q5_1", "Q8_0", "Q4K", "Q5K", "Q6K", "F16", "BF16"):
        cases += [("cfg2", QT[name], 18944, 3584, 2), ("cfg2", QT[name], 3584, 18944, 2)]
    out = []
    for cfg, ty, rows, cols, seed in cases:
        data = llrs.blocks.random_tensor_bytes(ty, rows, cols, seed=seed)
        nbytes = len(data)
        # Enough copies that the MALL cannot serve a repeat (the floor cases: two).
        copies = 2 if cfg == "floor" else max(2, int(1.2e9 // nbytes) + 1)
        qt = llrs.QuantTensor(data, (rows, cols), ty)
        ts = [be.upload(qt) for _ in range(copies)]
        x, y = C.c_void_p(), C.c_void_p()
        llrs._check(lib.llrs_device_alloc(be.handle, cols * 4, C.byref(x)))
        llrs._check(lib.llrs_device_alloc(be.handle, rows * 4, C.byref(y)))
        try:
            xs = llrs.blocks.random_activation(cols, seed)
            llrs._check(lib.llrs_copy_h2d(be.handle, x, xs.ctypes.data, cols * 4))
            for t in ts:
                llrs._check(lib.llrs_matvec_dev(be.handle, t.handle, x, y))
            be.synchronize()
            n = max(2 * copies, min(2000, int(0.2 / (nbytes / 5e12))))  # ~0.2 s, at most 2000
            t0 = time.perf_counter()
            for i in range(n):
                lib.llrs_matvec_dev(be.handle, ts[i % copies].handle, x, y)
            be.synchronize()
            dt = (time.perf_counter() - t0) / n
        finally:
            lib.llrs_device_free(be.handle, x)
            lib.llrs_device_free(be.handle, y)
            del ts
        alg = nbytes + 4 * (rows + cols)
        rec = {"config": cfg, "type": ty.name, "rows": rows, "cols": cols, "weight_bytes": nbytes,
               "kernel": "tuned" if ty.name in TUNED_TYPES else "float" if ty.name in FLOAT_TYPES else "generic", "launches": n,
               "copies": copies, "us": round(dt * 1e6, 2), "gbs": round(alg / dt / 1e9, 1),
               "frac": round(alg / dt / 1e9 / PEAK_HBM_GBS, 4)}
        log(f"{cfg} {ty.name:5s} {rows:6d} x {cols:5d} {nbytes / 1e6:8.2f} MB {rec['kernel']:7s} "
            f"{rec['us']:9.2f} us {rec['gbs']:7.1f} GB/s ({100 * rec['frac']:.1f}% of peak)")
        if oracle is not None:
            cpu = {"kind": "port", "reps": cpu_reps, "statistic": "median"}
            for name, kernel, th in (("avx2_all", AVX2, threads), ("avx2_one", AVX2, 1),
                                     ("scalar_all", SCALAR, threads)):
                dt_c = gemv_cpu(oracle, kernel, th, data, int(ty), rows, cols, xs, cpu_reps)
                cpu[name] = {"us": round(dt_c * 1e6, 1), "gbs": round(alg / dt_c / 1e9, 2), "threads": th}
            rec["cpu_baseline"] = cpu
            log(f"  cpu: AVX2 {cpu['avx2_all']['gbs']} GB/s on {threads} threads, "
                f"{cpu['avx2_one']['gbs']} on 1; scalar {cpu['scalar_all']['gbs']} on {threads}; "
                f"GPU / AVX2-all {rec['gbs'] / cpu['avx2_all']['gbs']:.0f}x")
        out.append(rec)
    print(json.dumps({"gemv": out}), flush=True)
    return 0


def profiled_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE, each scaled by the calibration copy) and the
    commit its runs measured, or (None, None)."""
    f = ROOT / "profiles" / "pmc_traffic_7b_q4km.md"
    if not f.exists():
        return None, None
    nbytes = commit = None
    for line in f.read_text().splitlines():
        parts = line.strip().strip("`").split()
        if len(parts) == 3 and parts[0] == "traffic_bytes_per_launch" and parts[1] == kernel:
            nbytes = int(parts[2])
        if len(parts) == 3 and parts[0] == "traffic_commit" and parts[1] == kernel:
            commit = parts[2]
    return nbytes, commit


# The end-to-end benchmark configs: synthetic models (random-init
# N(0, 0.02) weights, quantized in HBM), prompt length and decode steps.
# cfg5 is the headline (the default); cfg3 and cfg4 are run on request.
WORKLOADS = {
    "cfg5": dict(metric=METRIC, prompt=512, steps=128, recipe="Q4KM", seed=5,
                 desc="cfg5: Qwen2.5-7B-shape q4km, 512-token prefill then batch-1 greedy decode",
                 shape=dict(hidden_size=3584, intermediate_size=18944, num_attention_heads=28,
                            num_key_value_heads=4, num_hidden_layers=28, vocab_size=152064,
                            tie_word_embeddings=False)),
    "cfg3": dict(metric="batch-1 decode tok/s + achieved HBM GB/s (% of peak), Qwen2.5-0.5B-shape q4km",
                 prompt=128, steps=32, recipe="Q4KM", seed=3,
                 desc="cfg3: Qwen2.5-0.5B-shape q4km (Q5_0 fallback for 896-wide rows, tied "
                      "embeddings), 128-token prefill then 32 greedy decode steps",
                 shape=dict(hidden_size=896, intermediate_size=4864, num_attention_heads=14,
                            num_key_value_heads=2, num_hidden_layers=24, vocab_size=151936,
                            tie_word_embeddings=True)),
    "cfg4": dict(metric="batch-1 decode tok/s + achieved HBM GB/s (% of peak), Qwen2.5-1.5B-shape q4k "
                        "at KV depth 4000",
                 prompt=4000, steps=64, recipe="Q4K", seed=4,
                 desc="cfg4: Qwen2.5-1.5B-shape uniform q4k (tied embeddings), KV cache prefilled to "
                      "depth 4000 with random tokens, then 64 greedy decode steps",
                 shape=dict(hidden_size=1536, intermediate_size=8960, num_attention_heads=12,
                            num_key_value_heads=2, num_hidden_layers=28, vocab_size=151936,
                            tie_word_embeddings=True)),
}


HF_LAYER_TENSORS = (  # (name, rows, cols) per layer; "H", "F", "KV" stand for the widths
    ("input_layernorm.weight", None, "H"), ("post_attention_layernorm.weight", None, "H"),
    ("self_attn.q_proj.weight", "H", "H"), ("self_attn.q_proj.bias", None, "H"),
    ("self_attn.k_proj.weight", "KV", "H"), ("self_attn.k_proj.bias", None, "KV"),
    ("self_attn.v_proj.weight", "KV", "H"), ("self_attn.v_proj.bias", None, "KV"),
    ("self_attn.o_proj.weight", "H", "H"), ("mlp.gate_proj.weight", "F", "H"),
    ("mlp.up_proj.weight", "F", "H"), ("mlp.down_proj.weight", "H", "F"))


def write_hf_checkpoint(shape: dict, out: pathlib.Path, seed: int) -> int:
    """A Hugging Face BF16 checkpoint (config.json + model.safetensors) of the
    workload's shape, its values tiled from a 32 MiB block of N(0, 0.02)
    bf16 draws (norm gains 1 + N(0, 0.02)); returns the file's size."""
    H, F, L, V = (shape[k] for k in ("hidden_size", "intermediate_size", "num_hidden_layers",
                                     "vocab_size"))
    KV = shape["num_key_value_heads"] * (H // shape["num_attention_heads"])
    dims = {"H": H, "F": F, "KV": KV}
    tensors = [("model.embed_tokens.weight", (V, H)), ("model.norm.weight", (H,))]
    for i in range(L):
        tensors += [(f"model.layers.{i}.{n}", (dims[c],) if r is None else (dims[r], dims[c]))
                    for n, r, c in HF_LAYER_TENSORS]
    if not shape["tie_word_embeddings"]:
        tensors.append(("lm_head.weight", (V, H)))
    header, off = {"__metadata__": {"format": "pt"}}, 0
    for name, shp in tensors:
        n = int(np.prod(shp)) * 2
        header[name] = {"dtype": "BF16", "shape": list(shp), "data_offsets": [off, off + n]}
        off += n
    hdr = json.dumps(header).encode()
    hdr += b" " * (-len(hdr) % 8)
    rng = np.random.default_rng(seed)
    block = (rng.standard_normal(16 << 20).astype(np.float32) * 0.02).view(np.uint32)
    block = ((block + 0x8000) >> 16).astype(np.uint16)  # round to nearest bf16
    gain = ((((1 + rng.standard_normal(65536).astype(np.float32) * 0.02).view(np.uint32)
              + 0x8000) >> 16).astype(np.uint16))
    with open(out / "model.safetensors", "wb") as f:
        f.write(len(hdr).to_bytes(8, "little") + hdr)
        for name, shp in tensors:
            n = int(np.prod(shp))
            src = gain if name.endswith("norm.weight") else block
            while n:
                k = min(n, src.size)
                f.write(src[:k].tobytes())
                n -= k
    config = {"model_type": "qwen2", "architectures": ["Qwen2ForCausalLM"],
              "max_position_embeddings": 32768, "rms_norm_eps": 1e-6, "rope_theta": 1e6,
              "torch_dtype": "bfloat16", **shape}
    (out / "config.json").write_text(json.dumps(config))
    return 8 + len(hdr) + off


def load_bench(llrs, be, workload: str, cpu_seconds: float, keep: bool) -> int:
    """SafetensorsLoader::load with load-time q4km quantization: a BF16
    checkpoint of the workload's shape is written to a temporary directory,
    loaded once untimed (page cache, code objects) and once timed.  `value`
    is checkpoint bytes / load seconds; the CPU baseline is the host encoder
    (the reference's sequential quantize_* loops, one thread) on a bounded
    sample of the same matrices."""
    import shutil
    import tempfile
    wl = WORKLOADS[workload]
    d = pathlib.Path(tempfile.mkdtemp(prefix="llrs_ckpt_", dir=os.environ.get("TMPDIR", "/tmp")))
    try:
        t0 = time.perf_counter()
        nbytes = write_hf_checkpoint(wl["shape"], d, wl["seed"])
        log(f"wrote a {nbytes / 1e9:.2f} GB BF16 checkpoint in {time.perf_counter() - t0:.1f}s")
        times = []
        for i in range(2):
            t0 = time.perf_counter()
            model = llrs.ModelLoader.load(d, be, llrs.LoadQuantization.Q4KM)
            be.synchronize()
            times.append(time.perf_counter() - t0)
            wbytes = model.weight_bytes()
            log(f"load {i} ({'timed' if i else 'warm-up'}): {times[-1]:.2f}s")
            if i == 0:
                del model
        kv = llrs.KVCache(model, 64)
        model.prefill(np.arange(8, dtype=np.uint32), 0, kv)
        toks = model.decode_greedy(8, 4, kv)
        log(f"loaded model decodes: {toks.tolist()}")
        # Host encoder on a sample of the same matrices (gate_proj rows).
        H, F = wl["shape"]["hidden_size"], wl["shape"]["intermediate_size"]
        rng = np.random.default_rng(wl["seed"])
        vals = rng.standard_normal((256, H)).astype(np.float32) * 0.02
        rows, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < min(cpu_seconds, 10.0):
            llrs.QuantTensor.quantize(llrs.QuantType.Q4K, vals, 256, H)
            rows += 256
        cpu_s = time.perf_counter() - t0
        cpu_gbs = rows * H * 2 / cpu_s / 1e9
        rec = {"metric": "load-time q4km quantization of a BF16 safetensors checkpoint",
               "value": round(nbytes / times[1] / 1e9, 3), "unit": "GB/s of checkpoint",
               "load_s": round(times[1], 3), "checkpoint_bytes": nbytes,
               "weight_bytes_per_token_after": wbytes, "higher_is_better": True,
               "dtype": "bf16->q4km", "data": "synthetic",
               "config": {"workload": f"{workload} shape, HF BF16 -> q4km (Q4_K/Q8_0/Q6_K)"},
               "cpu_baseline": {"value": round(cpu_gbs, 4), "unit": "GB/s of checkpoint",
                                "cores": 1, "kind": "port",
                                "sample": f"{rows} rows x {H} of Q4_K (gate_proj-shaped), host encoder"},
               "cpu_projected_load_s": round(nbytes / (cpu_gbs * 1e9), 1)}
        print(json.dumps(rec), flush=True)
    finally:
        if keep:
            log(f"kept {d}")
        else:
            shutil.rmtree(d, ignore_errors=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="cfg5")
    ap.add_argument("--steps", type=int, default=None, help="timed decode steps (workload default)")
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--rounds", type=int, default=3, help="timed benchmark_tokens rounds (median)")
    ap.add_argument("--prompt", type=int, default=None, help="prompt tokens (workload default)")
    ap.add_argument("--context", type=int, default=4096)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--profile-iters", type=int, default=5)
    ap.add_argument("--projection-only", choices=["qkv", "o", "gate_up", "down", "lm_head", "layers"],
                    help="only time this projection's launches over all layers and run the "
                         "calibration copy (the workload of the rocprofv3 --pmc traffic runs)")
    ap.add_argument("--gemv", action="store_true",
                    help="configs 1 and 2 instead: single GEMVs per type over rotating weight copies")
    ap.add_argument("--lds-probe", type=int, default=0, metavar="ITERS",
                    help="instead: the LDS bank-pattern probe kernels, ITERS accesses per thread")
    ap.add_argument("--lds-probe-reps", type=int, default=1,
                    help="--lds-probe: launches of each probe kernel")
    ap.add_argument("--gemv-cpu-reps", type=int, default=20,
                    help="--gemv: host oracle calls per case and path (median; 0 = no CPU timing)")
    ap.add_argument("--load", action="store_true",
                    help="instead: load a BF16 safetensors checkpoint of the workload's shape with "
                         "load-time q4km quantization")
    ap.add_argument("--keep-checkpoint", action="store_true", help="--load: keep the written files")
    args = ap.parse_args()
    wl = WORKLOADS[args.workload]
    if args.steps is None:
        args.steps = wl["steps"]
    if args.prompt is None:
        args.prompt = wl["prompt"]
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported "
              "(this build has no multi-GPU path)", file=sys.stderr)
        return 2
    if args.prompt + args.warmup + args.steps > args.context:
        print("prompt + warmup + steps exceed the context", file=sys.stderr)
        return 2

    llrs = package()
    be = llrs.HipBackend(0)
    log(f"backend {be.name()} with {be.threads()} CUs")
    if args.lds_probe:
        return lds_probe(llrs, be, args.lds_probe, args.lds_probe_reps)
    if args.gemv:
        return gemv_sweep(llrs, be, 0 if args.no_cpu_baseline else args.gemv_cpu_reps)
    if args.load:
        return load_bench(llrs, be, args.workload, args.cpu_seconds, args.keep_checkpoint)
    cfg = llrs.SynthConfig(max_position_embeddings=32768, rope_theta=1e6, rms_norm_eps=1e-6,
                           recipe=getattr(llrs.LoadQuantization, wl["recipe"]), seed=wl["seed"],
                           **wl["shape"])
    t0 = time.perf_counter()
    model = llrs.HipQwen2Model.synthetic(be, cfg)
    gen_s = time.perf_counter() - t0
    mc = model.config()
    wbytes = model.weight_bytes()
    log(f"generated the {args.workload} model in HBM in {gen_s:.1f}s: {wbytes / 1e9:.3f} GB of "
        f"weights/token")

    if args.projection_only:
        return projection_only(llrs, be, model, args.projection_only, args.profile_iters)

    engine = llrs.InferenceEngine(model, args.context)
    kv = engine.kv_cache
    prompt = np.random.default_rng(wl["seed"]).integers(0, mc.vocab_size, args.prompt).astype(np.uint32)
    # llama-bench's protocol (src/bin/llama-bench.rs:113-126): an untimed
    # benchmark_tokens of the prompt's first 8 tokens and 1 decode step, then
    # `rounds` timed benchmark_tokens (reset, prefill, `steps` greedy decode
    # steps; src/engine.rs:189-223), and the round that is the median by
    # prefill + decode time.  One more untimed round with `--warmup` decode
    # steps comes first (the prefill buffers' allocation, graph capture).
    engine.benchmark_tokens(prompt[:8], 1)
    engine.benchmark_tokens(prompt, args.warmup)
    results = []
    for _ in range(args.rounds):
        be.synchronize()
        results.append(engine.benchmark_tokens(prompt, args.steps))
    results.sort(key=lambda r: r.prefill_s + r.decode_s)
    med = results[len(results) // 2]
    prefill_s, dt, toks = med.prefill_s, med.decode_s, med.tokens
    pf_flops = prefill_flops(mc, args.prompt)
    log(f"rounds (prefill ms, decode ms): "
        + ", ".join(f"({r.prefill_s * 1e3:.1f}, {r.decode_s * 1e3:.1f})" for r in results))
    log(f"prefill {args.prompt} tokens in {prefill_s * 1e3:.1f} ms ({args.prompt / prefill_s:.1f} tok/s, "
        f"{pf_flops / prefill_s / 1e12:.1f} TFLOP/s = {100 * pf_flops / prefill_s / PEAK_F16_FLOPS:.2f}% "
        f"of the f16 MFMA peak)")
    tps = args.steps / dt
    pos0 = args.prompt
    bytes_tok = wbytes + sum(kv_bytes_per_token(mc, p) for p in range(pos0, pos0 + args.steps)) / args.steps
    hbm_gbs = bytes_tok * tps / 1e9
    log(f"decode {args.steps} steps in {dt * 1e3:.1f} ms: {tps:.1f} tok/s, "
        f"{hbm_gbs:.0f} GB/s ({100 * hbm_gbs / PEAK_HBM_GBS:.1f}% of peak); "
        f"first tokens {list(toks[:6])}")
    llama_bench = {"architecture": model.architecture(), "backend": be.name(), "threads": be.threads(),
                   "load_ms": round(gen_s * 1e3, 3), "prompt_tokens": args.prompt,
                   "prefill_ms": round(prefill_s * 1e3, 3), "prefill_tps": round(args.prompt / prefill_s, 3),
                   "decode_tokens": args.steps, "decode_ms": round(dt * 1e3, 3),
                   "decode_tps": round(tps, 3)}

    # On-device sampling (sample_current_logits, src/engine.rs:253-325) of the
    # last logits with the engine's default options: host-synchronous calls.
    sampler = llrs.Sampler(llrs.SamplingOptions())
    sampler.sample(kv, 0.5)
    t0 = time.perf_counter()
    for i in range(20):
        sampler.remember(sampler.sample(kv, (i + 0.5) / 20))
    sample_us = (time.perf_counter() - t0) / 20 * 1e6
    log(f"sampling {sample_us:.1f} us per call (temperature 0.7, top-k 40, top-p 0.9, penalty 1.1, "
        f"vocab {mc.vocab_size})")

    # Per-projection launch timing (HIP events, the backend's stream), rotating
    # over all layers so every launch streams weights from HBM.
    per = {}
    for which in model.PROJECTIONS:
        us, nb = model.profile_projection(kv, which, args.profile_iters)
        launches = 1 if which == "lm_head" else mc.num_hidden_layers
        per[which] = {"avg_us": round(us, 2), "bytes": nb, "gbs": round(nb / us / 1e3, 1),
                      "us_per_token": round(us * launches, 1)}
        log(f"  {which:8s} {us:8.2f} us/launch  {nb / 1e6:8.2f} MB  {nb / us / 1e3:7.1f} GB/s")
    if kv.persistent:
        # The dominant kernel is the persistent one (every layer in one launch):
        # weights of all layers plus the KV rows its attention reads and writes.
        pos_now = pos0 + args.steps
        us, wb = model.profile_layers(kv, args.profile_iters)
        kvb = kv_bytes_per_token(mc, pos_now)
        per["layers"] = {"avg_us": round(us, 2), "bytes": wb + kvb,
                         "gbs": round((wb + kvb) / us / 1e3, 1), "us_per_token": round(us, 1)}
        log(f"  layers   {us:8.2f} us/launch  {(wb + kvb) / 1e6:8.2f} MB  {(wb + kvb) / us / 1e3:7.1f} GB/s "
            f"(persistent kernel, position {pos_now})")
        achieved = (wb + kvb) / us / 1e3
        traffic, commit = profiled_traffic("decode_persistent_kernel") if args.workload == "cfg5" else (None, None)
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                    "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                    "traffic": traffic,
                    "traffic_source": (f"profiles/pmc_traffic_7b_q4km.md: rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE "
                                       f"at commit {commit}") if traffic else None,
                    "kernel": f"decode_persistent_kernel: all {mc.num_hidden_layers} layers in one "
                              f"launch ({wb} weight bytes + {kvb} KV bytes at position {pos_now})"}
    else:
        dom = max(per, key=lambda k: per[k]["us_per_token"])
        d = per[dom]
        achieved = d["bytes"] / d["avg_us"] / 1e3
        traffic, commit = profiled_traffic(dom) if args.workload == "cfg5" else (None, None)
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                    "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                    "traffic": traffic,
                    "traffic_source": (f"profiles/pmc_traffic_7b_q4km.md: rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE "
                                       f"at commit {commit}") if traffic else None,
                    "kernel": f"{dom} projection GEMV ({d['bytes']} algorithmic weight bytes/launch)"}

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(llrs, model, kv, args.prompt, int(toks[0]), args.cpu_seconds,
                           f"{args.workload} {wl['recipe'].lower()}")
        log(f"cpu baseline {cpu['value']} tok/s on {cpu['cores']} threads, "
            f"{cpu['one_thread']['value']} on one, scalar {cpu['scalar']['value']}")

    out = {
        "metric": wl["metric"], "value": round(tps, 3), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(1e3 * dt / args.steps, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8x2 activation digits . q4km weight codes -> int32, f32 scales and sums",
        "data": f"synthetic (random-init N(0,0.02) weights, {wl['recipe'].lower()}-quantized in HBM; "
                "random prompt ids)",
        "config": {"workload": wl["desc"], "prompt_tokens": args.prompt, "decode_start_pos": pos0,
                   "context": args.context, "global_batch": 1, "parallelism": "none",
                   "protocol": f"llama-bench: warm-up, median of {args.rounds} rounds by prefill + decode"},
        "llama_bench": llama_bench,
        "hbm_gbps": round(hbm_gbs, 1), "hbm_pct_peak": round(100 * hbm_gbs / PEAK_HBM_GBS, 2),
        "sample_us": round(sample_us, 1),
        "bytes_per_token": int(bytes_tok), "prefill_tps": round(args.prompt / prefill_s, 2),
        "prefill": {"tokens": args.prompt, "ms": round(prefill_s * 1e3, 2),
                    "tflops": round(pf_flops / prefill_s / 1e12, 2),
                    "mfma_util": round(pf_flops / prefill_s / PEAK_F16_FLOPS, 4),
                    "peak": "2.5 PFLOP/s dense f16"},
        "model_gen_s": round(gen_s, 2), "roofline": roofline, "cpu_baseline": cpu,
        "projections": per,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
