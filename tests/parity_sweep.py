"""Randomized parity sweep of the sampler against the oracle (MI355X).

    python tests/parity_sweep.py START COUNT [--stop-on-mismatch]

Seeds START .. START+COUNT-1 each name a case (``tests.helpers.sweep_case``):
1-16 rows, bf16 / f16 / fp32, V from 7 to 151936, five value shapes,
per-row parameters, ragged histories, soft-caps.  Every row is sampled on
``cuda:0`` (token, keep mask, filtered values) and classified against the
oracle; rows with a status bit are counted apart.  A progress line every 25
seeds; the totals at the end.  Exit status 1 when a MISMATCH was found."""

from __future__ import annotations

import os
import sys
import time

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def main(argv) -> int:
    from tests.helpers import run_sweep_case

    start, count = int(argv[0]), int(argv[1])
    stop = "--stop-on-mismatch" in argv
    tot = {"rows": 0}
    bad = []
    t0 = time.time()
    for seed in range(start, start + count):
        w, ok_rows, st, summ, verdicts, _, _ = run_sweep_case(seed)
        tot["rows"] += w.batch
        for s in st.tolist():
            if s:
                tot[f"status_{s}"] = tot.get(f"status_{s}", 0) + 1
        for k, v in summ.items():
            if k != "max_margin":
                tot[k] = tot.get(k, 0) + v
        for b, v in zip(ok_rows, verdicts):
            if not v.ok:
                bad.append((seed, b, str(w.logits.dtype), w.vocab, v.details[:3]))
                print("MISMATCH", bad[-1], flush=True)
        if bad and stop:
            break
        if (seed - start + 1) % 25 == 0:
            print(f"seed {seed} {time.time() - t0:.0f}s {tot}", flush=True)
    print("TOTAL", tot, flush=True)
    print("MISMATCH cases", len(bad), flush=True)
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
