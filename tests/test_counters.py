"""The counter summariser reads rocprofv3 CSV passes and derives ratios."""

import csv

from rl_project_amd import counters

FIELDS = ["Correlation_Id", "Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]


def _write(path, rows):
    path.parent.mkdir(parents=True, exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, FIELDS)
        w.writeheader()
        for r in rows:
            w.writerow(dict(zip(FIELDS, r)))


def test_summary_of_two_passes(tmp_path):
    # 8 dispatches of the kernel (2 dropped as warm-up) and one other kernel;
    # a counter reported on two rows of a dispatch is summed
    p1, p2 = [], []
    for d in range(8):
        p1 += [(d, d, "k_sample_rows16<BF16>", "SQ_WAVES", 4096), (d, d, "k_sample_rows16<BF16>", "SQ_INSTS_VALU", 5e6),
               (d, d, "k_sample_rows16<BF16>", "SQ_INSTS_VALU", 5e6), (d, d, "other", "SQ_WAVES", 1)]
        p2 += [(d, d, "k_sample_rows16<BF16>", "TCC_EA0_RDREQ_sum", 100 + d),
               (d, d, "k_sample_rows16<BF16>", "TCC_EA0_RDREQ_32B_sum", 0),
               (d, d, "k_sample_rows16<BF16>", "TCC_EA0_RDREQ_64B_sum", 0),
               (d, d, "k_sample_rows16<BF16>", "TCC_EA0_RDREQ_128B_sum", 100 + d),
               (d, d, "k_sample_rows16<BF16>", "FETCH_SIZE", (100 + d) * 64 / 1024)]
    _write(tmp_path / "p1" / "x" / "run_counter_collection.csv", p1)
    _write(tmp_path / "p2" / "run_counter_collection.csv", p2)
    c = counters.load([str(tmp_path / "p1"), str(tmp_path / "p2")], "k_sample_rows16")
    assert c["SQ_WAVES"] == [4096] * 6 and c["SQ_INSTS_VALU"] == [1e7] * 6
    assert c["TCC_EA0_RDREQ_128B_sum"] == [102, 103, 104, 105, 106, 107]
    text = counters.summarise("k_sample_rows16", 64 * 1e6, [str(tmp_path / "p1"), str(tmp_path / "p2")])
    assert "SQ_INSTS_VALU per wave                       2441.4" in text
    assert "SQ_INSTS_VALU lane-instructions per element  10.00" in text
    assert "request-size bytes / FETCH_SIZE bytes        2.0000" in text
    assert "no dispatch" in counters.summarise("missing", 1, [str(tmp_path / "p1")])
