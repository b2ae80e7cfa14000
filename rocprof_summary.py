"""Summaries of rocprofv3 CSV output for the committed profiles.

  python rocprof_summary.py stats <kernel_stats.csv> [name-substring ...]
      per-kernel call count and average / min / max duration (µs), plus the
      call-weighted average over every kernel matching each substring
  python rocprof_summary.py trace <kernel_trace.csv> <name-substring> <last-N>
      duration of the last N dispatches whose kernel name contains the
      substring (the timed region of a bench run: its last steps x launches):
      average / min / max, the average gap from one such dispatch's end to
      the next one's start, and the span from the first start to the last
      end divided by N
  python rocprof_summary.py pmc <counter_collection.csv> <name-substring> <last-N>
      per-dispatch average of each counter over the last N dispatches whose
      kernel name contains the substring (counter instances summed)

Reads only the CSV files rocprofv3 --output-format csv writes.
"""
import collections
import csv
import sys


def stats(path, patterns):
    rows = list(csv.DictReader(open(path)))
    for r in rows:
        print(f"{r['Name'][:90]:90s} calls={r['Calls']:>6s} avg_us={float(r['AverageNs']) / 1e3:9.3f} "
              f"min_us={float(r['MinNs']) / 1e3:9.3f} max_us={float(r['MaxNs']) / 1e3:9.3f}")
    for pat in patterns:
        sel = [r for r in rows if pat in r["Name"]]
        calls = sum(int(r["Calls"]) for r in sel)
        total = sum(float(r["TotalDurationNs"]) for r in sel)
        if calls:
            print(f"weighted[{pat}] calls={calls} avg_us={total / calls / 1e3:.3f}")


def trace(path, pattern, last):
    rows = [r for r in csv.DictReader(open(path)) if pattern in r["Kernel_Name"]]
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    rows = rows[-last:]
    dur = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in rows]
    gaps = [(int(b["Start_Timestamp"]) - int(a["End_Timestamp"])) / 1e3 for a, b in zip(rows, rows[1:])]
    span = (int(rows[-1]["End_Timestamp"]) - int(rows[0]["Start_Timestamp"])) / 1e3
    print(f"dispatches={len(rows)} pattern={pattern}")
    print(f"avg_us={sum(dur) / len(dur):.3f} min_us={min(dur):.3f} max_us={max(dur):.3f}")
    if gaps:
        print(f"avg_gap_us={sum(gaps) / len(gaps):.3f} min_gap_us={min(gaps):.3f} max_gap_us={max(gaps):.3f}")
    print(f"span_per_dispatch_us={span / len(rows):.3f}")


def pmc(path, pattern, last):
    per = collections.defaultdict(lambda: collections.Counter())
    for r in csv.DictReader(open(path)):
        if pattern in r["Kernel_Name"]:
            per[int(r["Dispatch_Id"])][r["Counter_Name"]] += float(r["Counter_Value"])
    ids = sorted(per)[-last:]
    tot = collections.Counter()
    for d in ids:
        tot.update(per[d])
    print(f"dispatches={len(ids)} pattern={pattern}")
    for k in sorted(tot):
        print(f"{k}_per_dispatch={tot[k] / max(1, len(ids)):.1f}")


if __name__ == "__main__":
    if sys.argv[1] == "stats":
        stats(sys.argv[2], sys.argv[3:])
    elif sys.argv[1] == "trace":
        trace(sys.argv[2], sys.argv[3], int(sys.argv[4]))
    elif sys.argv[1] == "pmc":
        pmc(sys.argv[2], sys.argv[3], int(sys.argv[4]))
    else:
        sys.exit(__doc__)
