"""Write golden vectors by running the reference sampler file itself.

Run in the build container only (it needs the reference checkout):

    python tests/golden/make_golden.py /root/reference

The reference package cannot be imported as a package (its
``models/loading.py`` imports a module the checkout does not contain), but
``src/forgeline/models/generation/sampling.py`` imports only ``torch`` and
``typing``, so it is loaded here as a single file.  Only
``apply_sampling_filters`` (``sampling.py:16-53``) is exercised: its boundary
tie-group membership under the unstable ``torch.sort`` (``:46``) and its
ulp-level softmax/cumsum rounding are the parts no closed form pins.

Each case is stored as inputs (logits, parameters, per-row history) and the
reference's filtered ``[1, V]`` output per row (one call per row, as the
inference engine makes, ``inference/engine.py:119``).  Soft-cap is not part
of the reference sampler; the soft-cap case applies ``tanh(x/c)*c`` with torch
first and records the reference filter of that.
"""

from __future__ import annotations

import importlib.util
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "sampler_golden.npz")


def load_reference(root: str):
    path = os.path.join(root, "src", "forgeline", "models", "generation", "sampling.py")
    spec = importlib.util.spec_from_file_location("_ref_sampling_file", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def zipf_ids(gen: torch.Generator, n: int, V: int, s: float) -> torch.Tensor:
    ranks = torch.arange(1, V + 1, dtype=torch.float64)
    cdf = torch.cumsum(ranks ** (-s), 0)
    cdf /= cdf[-1].clone()
    u = torch.rand(n, generator=gen, dtype=torch.float64)
    return torch.searchsorted(cdf, u).clamp(max=V - 1).to(torch.int64)


def build_cases():
    cases = []
    g = torch.Generator().manual_seed(1234)

    # 1. the reference's 1x4 known-answer test (tests/unit/test_models.py:50-59)
    kat = torch.tensor([[1.0, 2.0, 3.0, 4.0]])
    for name, kw in [("kat_topk1", dict(top_k=1)), ("kat_topp05", dict(top_p=0.5)),
                     ("kat_minp05", dict(min_p=0.5)), ("kat_rep2", dict(repetition_penalty=2.0, hist=[3]))]:
        p = dict(temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, repetition_penalty=1.0, hist=[])
        p.update(kw)
        cases.append((name, kat.clone(), [p]))

    # 2. the CPU plumbing workload: fp32 B=4 V=512 N(0, 3^2), T .8, k 50, p .9,
    #    rp 1.1 over 32 uniform ids per row
    B, V = 4, 512
    x = torch.randn(B, V, generator=g) * 3.0
    rows = []
    for b in range(B):
        hist = torch.randint(0, V, (32,), generator=g).tolist()
        rows.append(dict(temperature=0.8, top_k=50, top_p=0.9, min_p=0.0, repetition_penalty=1.1, hist=hist))
    cases.append(("plumbing_f32_4x512", x, rows))

    # 3. uniform-parameter workload at small V: fp32 N(0, 2^2) + 1% spikes of +8
    B, V = 6, 4096
    x = torch.randn(B, V, generator=g) * 2.0
    spike = torch.rand(B, V, generator=g) < 0.01
    x = x + 8.0 * spike
    rows = []
    for b in range(B):
        hist = torch.randint(0, V, (512,), generator=g).tolist()
        rows.append(dict(temperature=0.7, top_k=50, top_p=0.95, min_p=0.05, repetition_penalty=1.15, hist=hist))
    cases.append(("uniform_f32_6x4096", x, rows))

    # 4. heterogeneous bf16 rows: tie-heavy, every filter combination
    B, V = 12, 4096
    x = (torch.randn(B, V, generator=g) * 2.5).to(torch.bfloat16)
    ks = [0, 1, 20, 50, 200, 0, 0, 0, 50, 0, 3, 0]
    ps = [0.9, 0.5, 0.95, 1.0, 0.7, 0.99, 0.6, 0.8, 0.93, 1.0, 0.97, 0.75]
    mps = [0.0, 0.02, 0.1, 0.0, 0.0, 0.02, 0.0, 0.1, 0.05, 0.0, 0.0, 0.0]
    ts = [1.0, 0.7, 1.3, 0.1, 1.5, 0.9, 1.1, 0.5, 1.0, 0.0, 0.8, 1.2]
    rows = []
    for b in range(B):
        hist = zipf_ids(g, 256, V, 1.1).tolist()
        rp = [1.0, 1.1, 1.3, 1.05, 1.2, 1.0, 1.15, 1.0, 1.25, 1.1, 1.0, 1.3][b]
        rows.append(dict(temperature=ts[b], top_k=ks[b], top_p=ps[b], min_p=mps[b], repetition_penalty=rp, hist=hist))
    cases.append(("hetero_bf16_12x4096", x, rows))

    # 5. soft-capped Zipf-shaped fp32 rows, top-p only (large nucleus)
    B, V = 4, 4096
    rows = []
    xs = []
    for b in range(B):
        ranks = torch.randperm(V, generator=g).to(torch.float32) + 1.0
        xs.append(-1.2 * torch.log(ranks) + 0.5 * torch.randn(V, generator=g))
        rows.append(dict(temperature=1.0, top_k=0, top_p=0.9, min_p=0.0, repetition_penalty=1.0, hist=[], softcap=30.0))
    cases.append(("softcap_zipf_f32_4x4096", torch.stack(xs), rows))

    # 6. massive ties: bf16 values on a coarse grid, top-p inside a tie group
    B, V = 4, 2048
    x = (torch.randint(-8, 9, (B, V), generator=g).to(torch.float32) * 0.5).to(torch.bfloat16)
    rows = [dict(temperature=1.0, top_k=0, top_p=pp, min_p=0.0, repetition_penalty=1.0, hist=[])
            for pp in (0.3, 0.5, 0.77, 0.9)]
    cases.append(("ties_bf16_4x2048", x, rows))
    return cases


def main(root: str) -> None:
    ref = load_reference(root)
    cases = build_cases()
    arrays = {}
    meta = {"torch": torch.__version__, "aten_cpu_capability": torch.backends.cpu.get_cpu_capability(),
            "source": "src/forgeline/models/generation/sampling.py:16-53", "cases": []}
    for name, x, rows in cases:
        outs = []
        for b, p in enumerate(rows):
            row = x[b:b + 1].clone()
            cap = p.get("softcap", 0.0)
            if cap > 0:
                row = torch.tanh(row / cap) * cap
            past = p["hist"] if p["repetition_penalty"] != 1.0 else None
            y = ref.apply_sampling_filters(row, p["temperature"], p["top_k"] or None, p["top_p"],
                                           p["min_p"] or None, p["repetition_penalty"], past)
            outs.append(y[0])
        out = torch.stack(outs)
        if x.dtype == torch.bfloat16:
            arrays[f"{name}/logits_bf16"] = x.view(torch.int16).numpy()
            arrays[f"{name}/filtered_bf16"] = out.view(torch.int16).numpy()
        else:
            arrays[f"{name}/logits_f32"] = x.numpy()
            arrays[f"{name}/filtered_f32"] = out.numpy()
        H = max([len(p["hist"]) for p in rows] + [1])
        hist = np.full((len(rows), H), -1, dtype=np.int64)
        for b, p in enumerate(rows):
            hist[b, :len(p["hist"])] = p["hist"]
        arrays[f"{name}/hist"] = hist
        params = np.array([[p["temperature"], p["top_k"], p["top_p"], p["min_p"], p["repetition_penalty"],
                            p.get("softcap", 0.0)] for p in rows], dtype=np.float64)
        arrays[f"{name}/params"] = params
        meta["cases"].append(name)
    arrays["meta_json"] = np.frombuffer(json.dumps(meta).encode(), dtype=np.uint8)
    np.savez_compressed(OUT, **arrays)
    print("wrote", OUT, os.path.getsize(OUT), "bytes;", meta)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
