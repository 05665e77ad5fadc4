"""Per-phase timing of the persistent decode kernel, from the timing build.

    python llama.rs_amd/build.py --stamps
    python llama.rs_amd/phase_profile.py [--workload cfg5|cfg4|cfg3] [--steps N]

Loads libllrs_hip_stamps.so (the product library with the persistent decode
kernel compiled with -DLLRS_STAMPS: thread 0 of every workgroup stores the
100 MHz wall clock when it is released from a barrier, when its activation is
staged in LDS, when its weight streaming ends and when it arrives at the
next barrier), builds the workload's synthetic model, prefills its prompt,
decodes, and prints for each of the five phases of a layer (averaged over the
layers, then the median over the last `--steps` decode steps), in
microseconds:

    span      first release of the phase -> last arrival (the phase's length)
    release   last arrival at the previous barrier -> first release (barrier latency)
    stage     median workgroup: release -> activation staged
    stream    median workgroup: staged -> streaming done
    tail      median workgroup: streaming done -> arrival (epilogue, store drain)
    skew      first -> last arrival
    late-XCD  the XCD whose workgroups arrive last, on average (workgroup w runs on XCD w % 8)

and the kernel's total per layer.  The stamps are stores of one thread per
workgroup at points the kernel passes anyway; the timing build runs the
product kernel's arithmetic unchanged.
"""
from __future__ import annotations

import argparse
import ctypes as C
import importlib.util
import json
import pathlib
import sys

import numpy as np

PKG = pathlib.Path(__file__).resolve().parent
PHASES = ("qkv", "attention", "o_proj", "gate_up", "down")
K_INTERVALS, K_WGS = 5 * 64, 512

WORKLOADS = {
    "cfg5": dict(hidden_size=3584, intermediate_size=18944, num_attention_heads=28,
                 num_key_value_heads=4, num_hidden_layers=28, vocab_size=152064,
                 tie_word_embeddings=False, recipe="Q4KM", seed=5, prompt=512),
    "cfg4": dict(hidden_size=1536, intermediate_size=8960, num_attention_heads=12,
                 num_key_value_heads=2, num_hidden_layers=28, vocab_size=151936,
                 tie_word_embeddings=True, recipe="Q4K", seed=4, prompt=4000),
    "cfg3": dict(hidden_size=896, intermediate_size=4864, num_attention_heads=14,
                 num_key_value_heads=2, num_hidden_layers=24, vocab_size=151936,
                 tie_word_embeddings=True, recipe="Q4KM", seed=3, prompt=128),
}


def load_stamps_package(lib=None):
    spec = importlib.util.spec_from_file_location(
        "llama_rs_amd", PKG / "__init__.py", submodule_search_locations=[str(PKG)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["llama_rs_amd"] = mod
    spec.loader.exec_module(mod)
    mod.LIB_PATH = pathlib.Path(lib) if lib else PKG / "libllrs_hip_stamps.so"
    if not mod.LIB_PATH.exists():
        raise FileNotFoundError(f"{mod.LIB_PATH} is missing: run build.py --stamps")
    return mod


def read_stamps(llrs, nwg: int, nlayers: int) -> np.ndarray:
    buf = np.zeros(K_INTERVALS * K_WGS * 4, np.uint64)
    f = llrs.lib().llrs_debug_stamps
    f.restype, f.argtypes = C.c_int, [C.c_void_p, C.c_size_t]
    if f(buf.ctypes.data, buf.nbytes) != 0:
        raise RuntimeError("reading the stamps failed")
    return buf.reshape(K_INTERVALS, K_WGS, 4)[:5 * nlayers, :nwg, :].astype(np.int64)


def analyse(ts: np.ndarray, nlayers: int) -> dict:
    """Per phase, averaged over the layers: microseconds (ticks are 10 ns)."""
    out = {}
    ns = 10.0
    for ph, name in enumerate(PHASES):
        rows = []
        for l in range(nlayers):
            k = 5 * l + ph
            rel, arr = ts[k, :, 0], ts[k, :, 3]
            span = (arr.max() - rel.min()) * ns
            release = (rel.min() - ts[k - 1, :, 3].max()) * ns if k > 0 else 0.0
            skew = (arr.max() - arr.min()) * ns
            if ph == 1:
                stage = stream = 0.0
                tail = np.median(arr - rel) * ns
            else:
                stage = np.median(ts[k, :, 1] - rel) * ns
                stream = np.median(ts[k, :, 2] - ts[k, :, 1]) * ns
                tail = np.median(arr - ts[k, :, 2]) * ns
            xcd = [np.mean(arr[x::8]) for x in range(8)]
            rows.append((span, release, stage, stream, tail, skew, int(np.argmax(xcd))))
        a = np.array(rows, np.float64)
        out[name] = dict(span=a[:, 0].mean() / 1e3, release=a[:, 1].mean() / 1e3,
                         stage=a[:, 2].mean() / 1e3, stream=a[:, 3].mean() / 1e3,
                         tail=a[:, 4].mean() / 1e3, skew=a[:, 5].mean() / 1e3,
                         late_xcd=int(np.bincount(a[:, 6].astype(int), minlength=8).argmax()))
    total = (ts[5 * nlayers - 1, :, 3].max() - ts[0, :, 0].min()) * ns / 1e3
    out["kernel_us_per_layer"] = total / nlayers
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--workload", default="cfg5", choices=sorted(WORKLOADS))
    ap.add_argument("--steps", type=int, default=8)
    ap.add_argument("--json", action="store_true")
    ap.add_argument("--lib", default=None, help="a timing build other than libllrs_hip_stamps.so")
    ap.add_argument("--dump", default=None, help="also save every step's raw stamps (.npy)")
    args = ap.parse_args()
    llrs = load_stamps_package(args.lib)
    w = dict(WORKLOADS[args.workload])
    n_prompt = w.pop("prompt")
    w["recipe"] = getattr(llrs.LoadQuantization, w["recipe"])
    be = llrs.HipBackend(0)
    cfg = llrs.SynthConfig(max_position_embeddings=32768, rope_theta=1e6, rms_norm_eps=1e-6, **w)
    model = llrs.HipQwen2Model.synthetic(be, cfg)
    kv = llrs.KVCache(model, 4096 if n_prompt < 4000 else 4200)
    if not kv.persistent:
        raise SystemExit("the persistent decode kernel was not selected for this workload")
    prompt = np.random.default_rng(cfg.seed).integers(0, cfg.vocab_size, n_prompt).astype(np.uint32)
    model.prefill(prompt, 0, kv)
    model.decode_greedy(n_prompt, 8, kv)  # warm
    pos = n_prompt + 8
    per_step, raw = [], []
    for _ in range(args.steps):
        model.decode_greedy(pos, 1, kv)
        pos += 1
        ts = read_stamps(llrs, be.threads(), cfg.num_hidden_layers)
        raw.append(ts)
        per_step.append(analyse(ts, cfg.num_hidden_layers))
    if args.dump:
        np.save(args.dump, np.stack(raw))
    res = {}
    for name in PHASES:
        res[name] = {k: float(np.median([s[name][k] for s in per_step])) for k in per_step[0][name]}
    res["kernel_us_per_layer"] = float(np.median([s["kernel_us_per_layer"] for s in per_step]))
    if args.json:
        print(json.dumps(res))
        return
    print(f"persistent decode kernel, {args.workload}, positions {n_prompt + 8}..{pos - 1}, "
          f"{be.threads()} workgroups; median of {args.steps} steps, mean over "
          f"{cfg.num_hidden_layers} layers, microseconds")
    print(f"| phase | span | release | stage | stream | tail | skew | late XCD |")
    print(f"|---|---|---|---|---|---|---|---|")
    tot = 0.0
    for name in PHASES:
        r = res[name]
        tot += r["span"] + r["release"]
        print(f"| {name} | {r['span']:.2f} | {r['release']:.2f} | {r['stage']:.2f} | {r['stream']:.2f} | "
              f"{r['tail']:.2f} | {r['skew']:.2f} | {r['late_xcd']} |")
    print(f"\nsum of spans + releases {tot:.2f} us per layer; kernel {res['kernel_us_per_layer']:.2f} us per layer")


if __name__ == "__main__":
    main()
