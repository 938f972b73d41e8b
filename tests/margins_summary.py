"""Markdown summary of the parity margins a GPU test run recorded.

Run the GPU tests with ``QMLP_MARGINS=<file>`` (every check appends one JSON line
``{test, what, kind, ratio}``, ratio = error / bar, passing at <= 1), then
``python tests/margins_summary.py <file>``.  Kind ``fp16-h-raw`` is information only (the
block-float output's distance from the fp16-h formula in bars, before the rounding-tie allowance);
every other kind passes at a ratio <= 1.
"""
import json
import sys


def summarize(path):
    """Per test and check kind: the worst ratio, the case it came from and the number of checks."""
    rows = [json.loads(line) for line in open(path) if line.strip()]
    worst, count = {}, {}
    for r in rows:
        key = (r["test"], r["kind"])
        count[key] = count.get(key, 0) + 1
        if key not in worst or r["ratio"] > worst[key]["ratio"]:
            worst[key] = r
    out = [f"{len(rows)} checks; worst ratio (error / bar) per test and check kind, highest first.", "",
           "| ratio | kind | case | test | checks |", "|---|---|---|---|---|"]
    for key, r in sorted(worst.items(), key=lambda kv: -kv[1]["ratio"]):
        out.append(f"| {r['ratio']:.4f} | {key[1]} | {r['what']} | `{key[0].split('::', 1)[-1]}` | {count[key]} |")
    return "\n".join(out)


if __name__ == "__main__":
    print(summarize(sys.argv[1]))
