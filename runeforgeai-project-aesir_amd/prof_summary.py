"""Summarizes a rocprofv3 --kernel-trace database (rocpd SQLite) per kernel: calls, average /
min / max duration in microseconds and share of total kernel time.

    python runeforgeai-project-aesir_amd/prof_summary.py <run_results.db> [title]
"""
import sqlite3
import sys


def summarize(db: str) -> str:
    c = sqlite3.connect(db)
    rows = c.execute("select name, count(*), avg(duration), min(duration), max(duration), sum(duration), "
                     "avg(vgpr_count), avg(lds_size), avg(grid_x), avg(workgroup_x) from kernels group by name "
                     "order by sum(duration) desc").fetchall()
    tot = sum(r[5] for r in rows) or 1
    out = [f"| kernel | calls | avg us | min us | max us | % time | vgpr | lds B | workgroups |",
           "|---|---:|---:|---:|---:|---:|---:|---:|---:|"]
    for r in rows:
        name = r[0] if len(r[0]) < 90 else r[0][:87] + "..."
        wgs = int(r[8] / max(r[9], 1))
        out.append(f"| `{name}` | {r[1]} | {r[2] / 1e3:.2f} | {r[3] / 1e3:.2f} | {r[4] / 1e3:.2f} | "
                   f"{100 * r[5] / tot:.1f} | {r[6]:.0f} | {r[7]:.0f} | {wgs} |")
    return "\n".join(out)


if __name__ == "__main__":
    print(summarize(sys.argv[1]))
