"""Format the parity records of ``tests/test_gpu_configs.py`` as a markdown table.

Usage (on a GPU box):
    AYAKA_PARITY_LOG=gpurun_out/parity.jsonl python -m pytest tests/test_gpu_configs.py -m gpu -q
    python tests/parity_report.py gpurun_out/parity.jsonl > profiles/parity.md
"""

import json
import sys

COLS = [("max_rel_err_significant", "max rel. err, |ref| >= 0.1 row max"),
        ("max_err_over_row_max", "max err / row max"),
        ("max_row_normwise_err", "max row normwise err"),
        ("max_rel_err_above_floor", "max rel. err above the 1e-3 row floor")]


def main(path: str) -> None:
    recs = [json.loads(line) for line in open(path)]
    print("# Parity at every BASELINE configuration point\n")
    print("Command: `AYAKA_PARITY_LOG=gpurun_out/parity.jsonl python -m pytest tests/test_gpu_configs.py -m gpu -q`,")
    print("then `python tests/parity_report.py gpurun_out/parity.jsonl`.\n")
    print("Each point runs the layer API at full size (`FP8Config` -> `apply`) on the configuration's")
    print("input distribution. Errors are over *all* output rows against the oracle's restatement")
    print("evaluated on the device (its quantized operands checked bit for bit against the CPU")
    print("oracle's quantizer over all rows where a quantizer runs), bf16 output against the")
    print("bf16-rounded oracle. One bf16 ulp is 2^-7 = 7.81e-3 relative at the bottom of a binade.")
    print("The last column is dominated by fp32 summation-order differences on elements that")
    print("cancel to near the floor; the test bound there is absolute (1e-3 of the row max).\n")
    print("| Point | M | N | K | quant bit-exact checked | " + " | ".join(c[1] for c in COLS) + " |")
    print("|---|---|---|---|---|" + "---|" * len(COLS))
    for r in recs:
        a = r["all_rows"]
        print(f"| {r['label']} | {r['m']} | {r['n']} | {r['k']} | {'yes' if r.get('quant_checked_bit_exact') else '-'} | "
              + " | ".join(f"{a[c[0]]:.2e}" for c in COLS) + " |")
    worst = {c[0]: max(r["all_rows"][c[0]] for r in recs) for c in COLS}
    print("\nWorst over all points: " + ", ".join(f"{c[1]} {worst[c[0]]:.2e}" for c in COLS) + ".")


if __name__ == "__main__":
    main(sys.argv[1])
