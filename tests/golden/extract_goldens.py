"""Extract the reference's recorded block-index counts into reference_counts.json.

Reads data files of the reference checkout (default /root/reference; run once
where it exists, commit the JSON).  Nothing here imports or runs reference code:
it parses the numbers the reference recorded.

  results/results.csv       exact rows (sampled == 0): live and tile elements at
                            128^2 / 64^2 / 32^2 / 16^2 for N = 4096
                            (src/polyattn/experiments/granularity.py writes it)
  results/reindex.csv       waste = elements / live under class-A transforms
                            (identity, residue-perm-s: src/polyattn/transforms.py:63-74)
                            at 32^2 and 16^2, N = 4096 (src/polyattn/experiments/reindex.py:14-15)
  results/predictions-d4.txt  exp0 element counts, dilated-8, N = 4096
  out.out                   exp6 elements under rp-s (N = 4096), exp7 tiles total / max per
                            query block under rp2/4/8, gate permuted 16x16 waste
  gpu/exp8_three_cells.py:65-72  recorded (tiles, runs) / (tiles, max) per cell
"""
import csv
import json
import pathlib
import re
import sys

REF = pathlib.Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
OUT = pathlib.Path(__file__).resolve().parent / "reference_counts.json"

# masks whose definition is data independent (DocPacked uses a seeded lognormal stream)
SUPPORTED = {"causal", "window-128", "window-256", "window-512", "window-1024", "window-4096",
             "dilated-2", "dilated-4", "dilated-8", "sinks4+win256", "sinks4+win1024",
             "local256+str8", "prefixlm-1024"}


def results_csv():
    rows = []
    with open(REF / "results/results.csv") as f:
        for r in csv.DictReader(f):
            if r["sampled"] != "0" or r["mask"] not in SUPPORTED:
                continue
            rows.append(dict(mask=r["mask"], N=int(r["N"]), live=int(r["live"]),
                             elements={g: int(float(r[f"cost_{g}x{g}"])) for g in (128, 64, 32, 16)}))
    return rows


def reindex_csv():
    rows = []
    with open(REF / "results/reindex.csv") as f:
        for r in csv.DictReader(f):
            t = r["transform"]
            if r["cls"] != "A" or r["mask"] not in SUPPORTED:
                continue
            if t == "identity":
                s = 1
            elif t.startswith("residue-perm-"):
                s = int(t.rsplit("-", 1)[1])
            else:
                continue
            rows.append(dict(mask=r["mask"], N=4096, s=s, BQ=int(r["BQ"]), A=int(r["A"]),
                             waste=float(r["waste"])))
    return rows


def predictions():
    txt = (REF / "results/predictions-d4.txt").read_text()
    num = lambda pat: int(re.search(pat, txt).group(1).replace(",", ""))  # noqa: E731
    return [dict(mask="dilated-8", N=4096, s=1, BQ=128, A=128, elements=num(r"identity 128x128 elements\s+([\d,]+)")),
            dict(mask="dilated-8", N=4096, s=1, BQ=16, A=16, elements=num(r"identity 16x16\s+elements\s+([\d,]+)")),
            dict(mask="dilated-8", N=4096, s=8, BQ=16, A=16,
                 elements=num(r"residue-perm-8 16x16 elements\s+([\d,]+)"))]


def out_out():
    lines = (REF / "out.out").read_text().splitlines()
    exp6, exp7, gate = [], [], []
    fold6 = {"dilated-8": 8, "dilated-4": 4, "local256+str8": 8}   # gpu/exp6_traffic_multiplier.py:45
    pat6 = re.compile(r"^\s*(dilated-8|dilated-4|local256\+str8) (\d+)x(\d+?)(\d{6,})\s+cv")
    for ln in lines:
        m = pat6.match(ln)
        if m:
            name, bq, rest, elems = m.group(1), int(m.group(2)), m.group(3), m.group(4)
            # the printed row glues A and the element count together ("128x1281310720"):
            # A is one of the swept tile widths (gpu/exp6_traffic_multiplier.py:47)
            for a in (128, 64, 32, 16):
                joined = rest + elems
                if joined.startswith(str(a)):
                    exp6.append(dict(mask=name, N=4096, s=fold6[name], BQ=bq, A=a,
                                     elements=int(joined[len(str(a)):])))
                    break
    case = None
    for ln in lines:
        m = re.match(r"^\s*N=(\d+) (\d+)x(\d+)\s", ln)
        if m:
            case = tuple(int(x) for x in m.groups())
            continue
        m = re.match(r"^\s*rp(\d+)\s+tot (\d+)\s+max (\d+)\s", ln)
        if m and case:
            exp7.append(dict(mask="local256+str8", N=case[0], BQ=case[1], A=case[2], s=int(m.group(1)),
                             tiles=int(m.group(2)), max_kv=int(m.group(3))))
    for ln in lines:
        m = re.match(r"^\s*(dilated-4|dilated-8)\s+waste ([\d.]+)\s+max abs err", ln)
        if m:
            gate.append(dict(mask=m.group(1), N=1024, s=int(m.group(1).split("-")[1]), BQ=16, A=16,
                             waste_3dp=float(m.group(2))))
    # de-duplicate (several jobs print the same tables)
    dedup = lambda rows: [dict(t) for t in dict.fromkeys(tuple(sorted(r.items())) for r in rows)]  # noqa: E731
    return dedup(exp6), dedup(exp7), dedup(gate)


def exp8_cells():
    # gpu/exp8_three_cells.py:65-72: (tiles, runs) at 128x128, (tiles, max per block) at 128x32
    return [dict(mask="sinks4+win256", N=1024, BQ=128, A=128, s=1, tiles=26, runs=12),
            dict(mask="sinks4+win256", N=1024, BQ=128, A=128, s=8, tiles=64, runs=8),
            dict(mask="local256+str8", N=1024, BQ=128, A=128, s=1, tiles=36, runs=8),
            dict(mask="local256+str8", N=1024, BQ=128, A=128, s=2, tiles=34, runs=15),
            dict(mask="local256+str8", N=2048, BQ=128, A=32, s=2, tiles=408, max_kv=40),
            dict(mask="local256+str8", N=2048, BQ=128, A=32, s=4, tiles=424, max_kv=34)]


def main():
    exp6, exp7, gate = out_out()
    data = dict(source="recorded outputs of the reference (see extract_goldens.py)",
                results_csv=results_csv(), reindex_csv=reindex_csv(), predictions=predictions(),
                exp6=exp6, exp7=exp7, gate_waste=gate, exp8=exp8_cells())
    OUT.write_text(json.dumps(data, indent=1) + "\n")
    print(f"wrote {OUT}: " + ", ".join(f"{k}={len(v)}" for k, v in data.items() if isinstance(v, list)))


if __name__ == "__main__":
    main()
