"""Summaries of rocprofv3 result databases (the SQLite "rocpd" output) for the MoE step kernels.

Used to turn a `rocprofv3 --kernel-trace --stats` run and two `--pmc` runs (FETCH_SIZE, then
WRITE_SIZE) of `bench.py` into per-workload kernel durations and HBM bytes per launch:

    python -m k3moe.rocpd --kt KT.db --fetch FETCH.db --write WRITE.db --copy-bytes N \\
        --labels tp8-b1,tp8-b8,tp8-b64 --json traffic.json > summary.md

The counters are calibrated on a plain device copy of --copy-bytes bytes in the same run
(`bench.py --copy-probe N`): factor = bytes the copy moves / what the counter reports for it.
Dispatches of the step kernel are split into workloads in launch order (bench.py runs its
workloads one after another; each workload has its own LDS size).
"""

from __future__ import annotations

import argparse
import json
import sqlite3
import statistics

STEP_KERNELS = ('k_moe_single', 'k_moe_decode')  # the one-launch step kernels (one token; up to 64)
# (kernel_table takes any kernels: python -m k3moe.rocpd --kt KT.db [--fetch .. --write .. --copy-bytes N]
#  --table k_latent,k_moe)
COPY_KERNEL = 'copyBuffer'


def _like(names) -> tuple[str, tuple]:
    names = (names,) if isinstance(names, str) else tuple(names)
    return '(' + ' or '.join(['name like ?'] * len(names)) + ')', tuple(f'%{n}%' for n in names)


def _runs(rows):
    """Group consecutive rows by their first field (the dispatch's LDS size)."""
    out = []
    for key, *rest in rows:
        if not out or out[-1][0] != key:
            out.append((key, []))
        out[-1][1].append(rest)
    return out


def kernel_durations(db: str, name=STEP_KERNELS) -> list[dict]:
    con = sqlite3.connect(db)
    cond, args = _like(name)
    rows = con.execute(f'select lds_size, duration from kernels where {cond} order by start', args).fetchall()
    out = []
    for lds, vals in _runs(rows):
        us = [v[0] / 1e3 for v in vals]
        out.append({'lds_bytes': lds, 'dispatches': len(us), 'avg_us': round(statistics.fmean(us), 2),
                    'median_us': round(statistics.median(us), 2), 'min_us': round(min(us), 2),
                    'max_us': round(max(us), 2)})
    return out


def top_kernels(db: str, n: int = 6) -> list[dict]:
    con = sqlite3.connect(db)
    rows = con.execute('select name, count(*), avg(duration), sum(duration) from kernels group by name '
                       'order by sum(duration) desc limit ?', (n,)).fetchall()
    return [{'kernel': r[0][:90], 'dispatches': r[1], 'avg_us': round(r[2] / 1e3, 2),
             'total_us': round(r[3] / 1e3, 1)} for r in rows]


def counter_kib(db: str, counter: str, name) -> list[tuple[int, int, float]]:
    """(lds size, grid size, summed counter value in KiB) per dispatch of kernels matching `name`."""
    con = sqlite3.connect(db)
    cond, args = _like(name)
    cond = cond.replace('name like', 'kernel_name like')
    rows = con.execute('select lds_block_size, grid_size, sum(value) from counters_collection '
                       f'where counter_name = ? and {cond} group by dispatch_id order by start',
                       (counter,) + args).fetchall()
    return [(r[0], r[1], float(r[2])) for r in rows]


def calibration(db: str, counter: str, copy_bytes: int) -> float:
    """Bytes per reported KiB: the copy probe is the copy dispatch with the largest counter value."""
    vals = [v for _, _, v in counter_kib(db, counter, COPY_KERNEL)]
    return copy_bytes / max(vals)


def step_counter(db: str, counter: str) -> list[dict]:
    rows = [(lds, v) for lds, _, v in counter_kib(db, counter, STEP_KERNELS)]
    return [{'lds_bytes': lds, 'dispatches': len(vals), 'kib_per_dispatch': round(statistics.median([v[0] for v in vals]), 1)}
            for lds, vals in _runs(rows)]


def _short(name: str) -> str:
    """A kernel's name without its namespace and arguments (k3moe::k_latent<0>(...) -> k_latent<0>)."""
    return name.split('(')[0].replace('void ', '').replace('k3moe::', '')


def kernel_table(kt: str, fetch: str | None, write: str | None, names, copy_bytes: int | None) -> list[dict]:
    """Per (kernel, LDS size) group of dispatches in launch order, for kernels whose name contains
    one of `names`: median and mean duration and, with the counter runs, the median HBM read and
    write bytes per dispatch (FETCH_SIZE and WRITE_SIZE calibrated on the copy probe)."""
    con = sqlite3.connect(kt)
    cond, args = _like(names)
    groups: dict = {}
    for name, lds, dur in con.execute(f'select name, lds_size, duration from kernels where {cond} order by start', args):
        groups.setdefault((_short(name), lds), []).append(dur / 1e3)
    counters = {}
    for db, counter in ((fetch, 'FETCH_SIZE'), (write, 'WRITE_SIZE')):
        if not db:
            continue
        f = calibration(db, counter, copy_bytes)
        c = sqlite3.connect(db)
        cn, ca = _like(names)
        cn = cn.replace('name like', 'kernel_name like')
        vals: dict = {}
        for kn, lds, v in c.execute('select kernel_name, lds_block_size, sum(value) from counters_collection '
                                    f'where counter_name = ? and {cn} group by dispatch_id order by start',
                                    (counter,) + ca):
            vals.setdefault((_short(kn), lds), []).append(v * f)
        counters[counter] = vals
    out = []
    for (name, lds), us in groups.items():
        row = {'kernel': name, 'lds_bytes': lds, 'dispatches': len(us), 'median_us': round(statistics.median(us), 2),
               'avg_us': round(statistics.fmean(us), 2)}
        for counter, key in (('FETCH_SIZE', 'read_bytes'), ('WRITE_SIZE', 'write_bytes')):
            v = counters.get(counter, {}).get((name, lds))
            if v:
                row[key] = round(statistics.median(v))
        out.append(row)
    return out


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split('\n')[0])
    ap.add_argument('--kt', required=True, help='rocpd database of the --kernel-trace --stats run')
    ap.add_argument('--fetch', help='rocpd database of the --pmc FETCH_SIZE run')
    ap.add_argument('--write', help='rocpd database of the --pmc WRITE_SIZE run')
    ap.add_argument('--copy-bytes', type=int, help='bytes of the copy probe (bench.py --copy-probe)')
    ap.add_argument('--labels', help='workload names, in launch order (the step-kernel summary)')
    ap.add_argument('--algorithmic', default='', help='algorithmic bytes per workload, comma separated')
    ap.add_argument('--json', help='write the per-workload traffic here (merged into an existing file)')
    ap.add_argument('--table', help='instead: a per (kernel, LDS size) table for kernels whose names contain '
                    'one of these comma-separated strings')
    a = ap.parse_args(argv)
    if a.table:
        print('| kernel | LDS bytes | dispatches | median us | avg us | HBM read MB | HBM write MB |')
        print('|---|---|---|---|---|---|---|')
        for r in kernel_table(a.kt, a.fetch, a.write, a.table.split(','), a.copy_bytes):
            rd = f"{r['read_bytes'] / 1e6:.1f}" if 'read_bytes' in r else '-'
            wr = f"{r['write_bytes'] / 1e6:.2f}" if 'write_bytes' in r else '-'
            print(f"| `{r['kernel']}` | {r['lds_bytes']} | {r['dispatches']} | {r['median_us']} | {r['avg_us']} | "
                  f"{rd} | {wr} |")
        print('\nKernels of the whole run by total time:\n')
        print('| kernel | dispatches | avg us | total us |')
        print('|---|---|---|---|')
        for r in top_kernels(a.kt):
            print(f"| `{r['kernel']}` | {r['dispatches']} | {r['avg_us']} | {r['total_us']} |")
        return
    if not (a.fetch and a.write and a.copy_bytes and a.labels):
        raise SystemExit('--fetch, --write, --copy-bytes and --labels are needed for the step-kernel summary')
    labels = a.labels.split(',')
    algo = [int(x) for x in a.algorithmic.split(',')] if a.algorithmic else [None] * len(labels)
    durs = kernel_durations(a.kt)
    ff = calibration(a.fetch, 'FETCH_SIZE', a.copy_bytes)
    fw = calibration(a.write, 'WRITE_SIZE', a.copy_bytes)
    fetch, write = step_counter(a.fetch, 'FETCH_SIZE'), step_counter(a.write, 'WRITE_SIZE')
    if not (len(durs) == len(fetch) == len(write) == len(labels)):
        raise SystemExit(f'workload count mismatch: trace {len(durs)}, fetch {len(fetch)}, write {len(write)}, '
                         f'labels {len(labels)}')
    table = {}
    print(f'Counter calibration on the copy probe ({a.copy_bytes} bytes read and written): '
          f'FETCH_SIZE x {ff / 1024:.3f} KiB per reported KiB, WRITE_SIZE x {fw / 1024:.3f}.\n')
    print('| workload | dispatches | avg us | median us | min us | max us | FETCH_SIZE KiB | WRITE_SIZE KiB '
          '| HBM read MB | HBM write MB | traffic MB | algorithmic MB | traffic / algorithmic |')
    print('|---|---|---|---|---|---|---|---|---|---|---|---|---|')
    for lab, d, f, w, al in zip(labels, durs, fetch, write, algo):
        rd, wr = f['kib_per_dispatch'] * ff, w['kib_per_dispatch'] * fw
        tr = rd + wr
        ratio = f'{tr / al:.3f}' if al else '-'
        print(f"| {lab} | {d['dispatches']} | {d['avg_us']} | {d['median_us']} | {d['min_us']} | {d['max_us']} | "
              f"{f['kib_per_dispatch']} | {w['kib_per_dispatch']} | {rd / 1e6:.1f} | {wr / 1e6:.2f} | {tr / 1e6:.1f} | "
              f"{al / 1e6 if al else '-'} | {ratio} |")
        table[lab] = {'kernel_avg_us': d['avg_us'], 'kernel_median_us': d['median_us'], 'read_bytes': round(rd),
                      'write_bytes': round(wr), 'traffic_bytes': round(tr), 'algorithmic_bytes': al}
    print('\nKernels of the whole run by total time:\n')
    print('| kernel | dispatches | avg us | total us |')
    print('|---|---|---|---|')
    for r in top_kernels(a.kt):
        print(f"| `{r['kernel']}` | {r['dispatches']} | {r['avg_us']} | {r['total_us']} |")
    if a.json:   # merged into the file's workloads when it exists (one run per workload)
        doc = {'fetch_bytes_per_kib': ff, 'write_bytes_per_kib': fw, 'workloads': {}}
        try:
            with open(a.json) as fh:
                doc['workloads'] = json.load(fh).get('workloads', {})
        except (OSError, ValueError):
            pass
        doc['workloads'].update(table)
        with open(a.json, 'w') as fh:
            json.dump(doc, fh, indent=1)
            fh.write('\n')


if __name__ == '__main__':
    main()
