"""Builds the parity table (markdown) from the JSON lines test_gpu_configs.py appends to the file
named by QMM_PARITY_LOG: one row per case with the floored maximum relative error (the asserted
bar), the unfloored maximum, how many outputs pass 1e-3 unfloored, the largest |ref| among them
and the largest absolute error, both as fractions of the output rms.

    python tests/parity_table.py gpurun_out/parity_errors.jsonl > profiles/parity_errors.md
"""
import json
import sys


def main(path):
    rows = [json.loads(l) for l in open(path) if l.strip()]
    print("| case | path | floored max rel (bar 1e-3) | unfloored max rel | outputs > 1e-3 unfloored | "
          "max abs(ref)/rms there | max abs err / rms |")
    print("|---|---|---|---|---|---|---|")
    for r in rows:
        print(f"| {r['case']} | {r.get('path') or ''} | {r['floored']:.3g} | {r['unfloored']:.3g} | "
              f"{r['n_over_1e-3']} of {r['n']} | {r['max_abs_ref_over_rms']:.2g} | {r['max_abs_err_over_rms']:.2g} |")
    worst = max(rows, key=lambda r: r["floored"])
    print()
    print(f"{len(rows)} cases; the largest floored error is {worst['floored']:.3g} ({worst['case']}); "
          f"{sum(r['n_over_1e-3'] for r in rows)} of {sum(r['n'] for r in rows)} outputs pass 1e-3 unfloored.")


if __name__ == "__main__":
    main(sys.argv[1])
