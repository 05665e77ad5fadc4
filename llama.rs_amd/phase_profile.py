"""Per-phase timing of the persistent decode kernel, from the timing build.

    python llama.rs_amd/build.py --stamps
    python llama.rs_amd/phase_profile.py [--workload cfg5|cfg4|cfg3] [--steps N]

Loads libllrs_hip_stamps.so (the product library with the persistent decode
kernel compiled with -DLLRS_STAMPS: thread 0 of every workgroup stores the
100 MHz wall clock at fixed points of each barrier interval), builds the
workload's synthetic model, prefills its prompt, decodes, and prints, averaged
over the layers, then the median over the last `--steps` decode steps, in
microseconds, for each of the three barrier intervals of a layer
(A: Q/K/V + attention + o_proj, B: gate/up, C: down):

    span      first release of the interval -> last arrival at its end barrier
    release   last arrival at the previous barrier -> first release (barrier latency)
    stage     median workgroup: release -> activation staged
    stream    median workgroup: staged -> streaming done
    tail      median workgroup: streaming done -> arrival (epilogue, store drain)
    skew      first -> last arrival
    late-XCD  the XCD whose workgroups arrive last, on average (workgroup w runs on XCD w % 8)

and for interval A the median workgroup's segments: Q/K/V stage, stream and
epilogue, the attention items, o_proj's wait for the heads' outputs plus
staging, its streaming and its tail; plus the kernel's total per layer.  The
stamps are stores of one thread per workgroup at points the kernel passes
anyway; the timing build runs the product kernel's arithmetic unchanged.
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
PHASES = ("A_qkv_attn_o", "gate_up", "down")
SEGMENTS = ("qkv_stage", "qkv_stream", "qkv_epilogue", "attention", "o_wait_stage", "o_stream", "o_tail")
K_INTERVALS, K_WGS, K_SLOTS = 3 * 64, 512, 8
PER_LAYER = len(PHASES)

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
    buf = np.zeros(K_INTERVALS * K_WGS * K_SLOTS, np.uint64)
    f = llrs.lib().llrs_debug_stamps
    f.restype, f.argtypes = C.c_int, [C.c_void_p, C.c_size_t]
    if f(buf.ctypes.data, buf.nbytes) != 0:
        raise RuntimeError("reading the stamps failed")
    return buf.reshape(K_INTERVALS, K_WGS, K_SLOTS)[:PER_LAYER * nlayers, :nwg, :].astype(np.int64)


K_ITEMS = 4096


def read_item_stamps(llrs, nlayers: int) -> np.ndarray:
    buf = np.zeros(64 * K_ITEMS * 2, np.uint64)
    f = llrs.lib().llrs_debug_item_stamps
    f.restype, f.argtypes = C.c_int, [C.c_void_p, C.c_size_t]
    if f(buf.ctypes.data, buf.nbytes) != 0:
        raise RuntimeError("reading the item stamps failed")
    return buf.reshape(64, K_ITEMS, 2)[:nlayers].astype(np.int64)


def analyse_items(ts: np.ndarray, its: np.ndarray, nlayers: int, pos: int, nh: int, nkv: int) -> dict:
    """Interval A's attention items relative to the interval's first release:
    the median and last item start, the last end of non-merging items, and
    the median and last end of the merging (last-chunk) items (us)."""
    G, span = nh // nkv, 1
    n_pairs = nkv * (pos // 32 + 1)
    n_items = (n_pairs + 7) // 8 * 8 * G
    it = np.arange(n_items)
    r = it >> 3
    pair = (r // G) * 8 + (it & 7)
    live = pair < n_pairs
    chunk = pair // nkv
    last = chunk == pos // 32
    rows = []
    for l in range(nlayers):
        t0 = ts[PER_LAYER * l, :, 0].min()
        st, en = its[l, :n_items, 0], its[l, :n_items, 1]
        ok = live & (st > 0)
        if not ok.any():
            continue
        rows.append((np.median(st[ok] - t0), (st[ok] - t0).max(), (en[ok & ~last] - t0).max() if (ok & ~last).any() else 0,
                     np.median(en[ok & last] - t0), (en[ok & last] - t0).max()))
    a = np.array(rows, np.float64) * 10.0 / 1e3
    return dict(item_start_med=a[:, 0].mean(), item_start_max=a[:, 1].mean(), partial_end_max=a[:, 2].mean(),
                merge_end_med=a[:, 3].mean(), merge_end_max=a[:, 4].mean())


def analyse(ts: np.ndarray, nlayers: int) -> dict:
    """Per interval, averaged over the layers: microseconds (ticks are 10 ns)."""
    out = {}
    ns = 10.0
    for ph, name in enumerate(PHASES):
        rows = []
        for l in range(nlayers):
            k = PER_LAYER * l + ph
            rel, arr = ts[k, :, 0], ts[k, :, 3]
            span = (arr.max() - rel.min()) * ns
            release = (rel.min() - ts[k - 1, :, 3].max()) * ns if k > 0 else 0.0
            skew = (arr.max() - arr.min()) * ns
            stage = np.median(ts[k, :, 1] - rel) * ns
            stream = np.median(ts[k, :, 2] - ts[k, :, 1]) * ns
            tail = np.median(arr - (ts[k, :, 7] if ph == 0 else ts[k, :, 2])) * ns
            xcd = [np.mean(arr[x::8]) for x in range(8)]
            rows.append((span, release, stage, stream, tail, skew, int(np.argmax(xcd))))
        a = np.array(rows, np.float64)
        out[name] = dict(span=a[:, 0].mean() / 1e3, release=a[:, 1].mean() / 1e3,
                         stage=a[:, 2].mean() / 1e3, stream=a[:, 3].mean() / 1e3,
                         tail=a[:, 4].mean() / 1e3, skew=a[:, 5].mean() / 1e3,
                         late_xcd=int(np.bincount(a[:, 6].astype(int), minlength=8).argmax()))
    # Interval A's landmarks relative to its first release (us), mean over
    # layers: the last Q/K/V store, the median and last o_proj staging.
    lm = []
    for l in range(nlayers):
        t = ts[PER_LAYER * l]
        t0 = t[:, 0].min()
        lm.append(((t[:, 4] - t0).max(), np.median(t[:, 6] - t0), (t[:, 6] - t0).max(), (t[:, 3] - t0).max()))
    lm = np.array(lm, np.float64) * ns / 1e3
    out["landmarks_A"] = dict(qkv_stored_max=lm[:, 0].mean(), o_staged_med=lm[:, 1].mean(),
                              o_staged_max=lm[:, 2].mean(), arrival_max=lm[:, 3].mean())
    # Interval A's segments, median workgroup: slots 0 released, 1 staged, 2
    # streamed, 4 Q/K/V stored, 5 attention done, 6 o_proj staged, 7 o_proj
    # streamed, 3 arrival.
    seg = {n: [] for n in SEGMENTS}
    for l in range(nlayers):
        t = ts[PER_LAYER * l]
        for n, (a, b) in zip(SEGMENTS, ((0, 1), (1, 2), (2, 4), (4, 5), (5, 6), (6, 7), (7, 3))):
            seg[n].append(np.median(t[:, b] - t[:, a]) * ns)
    out["segments_A"] = {n: float(np.mean(v)) / 1e3 for n, v in seg.items()}
    total = (ts[PER_LAYER * nlayers - 1, :, 3].max() - ts[0, :, 0].min()) * ns / 1e3
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
        a = analyse(ts, cfg.num_hidden_layers)
        a["items_A"] = analyse_items(ts, read_item_stamps(llrs, cfg.num_hidden_layers), cfg.num_hidden_layers,
                                     pos - 1, cfg.num_attention_heads, cfg.num_key_value_heads)
        per_step.append(a)
    if args.dump:
        np.save(args.dump, np.stack(raw))
    res = {}
    for name in PHASES:
        res[name] = {k: float(np.median([s[name][k] for s in per_step])) for k in per_step[0][name]}
    res["segments_A"] = {n: float(np.median([s["segments_A"][n] for s in per_step])) for n in SEGMENTS}
    for key in ("landmarks_A", "items_A"):
        res[key] = {n: float(np.median([s[key][n] for s in per_step])) for n in per_step[0][key]}
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
    print("\ninterval A, median workgroup (us): " +
          ", ".join(f"{n} {res['segments_A'][n]:.2f}" for n in SEGMENTS))
    print("interval A, from its first release (us): " +
          ", ".join(f"{n} {v:.2f}" for n, v in {**res["landmarks_A"], **res["items_A"]}.items()))


if __name__ == "__main__":
    main()
