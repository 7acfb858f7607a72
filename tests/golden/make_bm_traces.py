"""Writes tests/golden/block_manager_traces.json: BlockManager operation scripts
and the outputs of the reference's own src/core/block_manager.cpp on them.

The reference implementation is compiled from its sources where they lie
(oracle/Makefile -> oracle/_ref/bm_trace_ref, driver oracle/bm_trace_driver.cpp);
this script only runs that binary.  Scripts are random but valid sequences
(no release or dec_ref of a free block, where this build deliberately differs):
acquire / release of singly-held blocks, inc/dec on held blocks, sequence
allocation, growth and freeing, capacity queries.

Run from the repository root after `make -C oracle`:  python tests/golden/make_bm_traces.py
"""
import json
import os
import random
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
REF = os.path.join(ROOT, "oracle", "_ref", "bm_trace_ref")
PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "block_manager_traces.json")


def make_script(seed: int, n_ops: int = 200) -> str:
    rng = random.Random(seed)
    bs = rng.choice([1, 4, 16, 32])
    ngpu = rng.choice([3, 8, 40, 257])
    ncpu = rng.choice([0, 4])
    lines = [f"new {bs} {ngpu} {ncpu}"]
    held = {}      # single blocks from acquire: id -> refcount
    tables = []    # live tables (index -> alive)
    free = ngpu
    for _ in range(n_ops):
        before = len(lines)
        op = rng.random()
        if op < 0.2:
            lines.append("acquire")
            # the driver output tells the id; the generator tracks it by replaying below
        elif op < 0.3 and held:
            bid = rng.choice(sorted(held))
            if held[bid] == 1:
                lines.append(f"release {bid}")
        elif op < 0.4 and held:
            bid = rng.choice(sorted(held))
            lines.append(f"inc {bid}")
        elif op < 0.5 and held:
            bid = rng.choice(sorted(held))
            lines.append(f"dec {bid}")
        elif op < 0.65:
            lines.append(f"alloc {rng.randint(0, bs * max(1, ngpu // 3))}")
        elif op < 0.8 and tables:
            t = rng.choice(tables)
            lines.append(f"ensure {t} {rng.randint(0, bs * max(1, ngpu // 2))}")
        elif op < 0.9 and tables:
            t = rng.choice(tables)
            lines.append(f"free {t}")
        elif op < 0.95:
            lines.append(f"can {rng.randint(0, ngpu + 2)}")
        else:
            lines.append("nfree")
        if len(lines) == before:
            continue
        # replay the script so far on the reference to keep the generator's state exact
        out = subprocess.run([REF], input="\n".join(lines) + "\n", capture_output=True, text=True,
                             check=True).stdout.split("\n")
        last, res = lines[-1], out[len(lines) - 1]
        parts = last.split()
        if parts[0] == "acquire" and res != "none":
            held[int(res)] = 1
        elif parts[0] == "release":
            held.pop(int(parts[1]), None)
        elif parts[0] == "inc":
            held[int(parts[1])] += 1
        elif parts[0] == "dec":
            held[int(parts[1])] -= 1
            if held[int(parts[1])] <= 0:
                held.pop(int(parts[1]))
        elif parts[0] == "alloc":
            tables.append(len([l for l in lines if l.startswith("alloc")]) - 1)
        elif parts[0] == "free":
            tables.remove(int(parts[1]))
    return "\n".join(lines) + "\n"


def main():
    if not os.path.exists(REF):
        raise SystemExit(f"{REF} missing: run make -C oracle (needs the reference tree)")
    cases = []
    for seed in range(12):
        script = make_script(seed, n_ops=60 + 20 * seed)
        out = subprocess.run([REF], input=script, capture_output=True, text=True, check=True).stdout
        cases.append({"seed": seed, "script": script, "expected": out})
    # the reference's own unit-test scenarios, as scripts
    cases.append({"seed": -1, "script": "new 16 10 0\nnfree\nacquire\nnfree\nrelease 9\nnfree\n",
                  "expected": subprocess.run([REF], input="new 16 10 0\nnfree\nacquire\nnfree\nrelease 9\nnfree\n",
                                             capture_output=True, text=True, check=True).stdout})
    with open(PATH, "w") as f:
        json.dump({"generator": "tests/golden/make_bm_traces.py", "reference": "src/core/block_manager.cpp",
                   "cases": cases}, f, indent=0)
    print(f"wrote {len(cases)} cases to {PATH}")


if __name__ == "__main__":
    main()
