"""Writes the prefix-mask-repair golden fixtures under tests/golden/repair/.

Each case is a tiny export directory in the layout the reference CLI reads
(src/tensor_group_prefix_mask_repair.cpp:219-249 manifest.csv, :251-292
analysis/plots/grouping_summary.csv, :294-326 raw little-endian tensor files),
plus the three reports the reference CLI, compiled from the reference sources
by oracle/Makefile into oracle/_ref/, writes for it (:477-604), stored under
expected/.  Run from the repository root after `make -C oracle`:

    python tests/golden/make_repair_fixtures.py

The inputs are committed, so the fixtures do not depend on this script's RNG.
"""
import os
import shutil
import subprocess
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
OUT = os.path.join(ROOT, "tests", "golden", "repair")
CLI = os.path.join(ROOT, "oracle", "_ref", "tensor_group_prefix_mask_repair")


def bf16(x):
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)   # round to nearest even
    return r


def write_case(name, tensors, groups, args):
    """tensors: list of (state_type, category, layer, dtype, uint16/uint32 array);
    groups: list of (state_type, category, group_id, layers, representative)."""
    d = os.path.join(OUT, name)
    shutil.rmtree(d, ignore_errors=True)
    os.makedirs(os.path.join(d, "tensors"))
    os.makedirs(os.path.join(d, "analysis", "plots"))
    with open(os.path.join(d, "manifest.csv"), "w") as f:
        f.write("tensor_key,layer,category,state_type,numel,dtype,file\n")
        for st, cat, layer, dt, arr in tensors:
            fn = f"tensors/{st}_{cat}_{layer}.bin"
            arr.astype(arr.dtype.newbyteorder("<")).tofile(os.path.join(d, fn))
            f.write(f"layers.{layer}.{cat}.{st},{layer},{cat},{st},{arr.size},{dt},{fn}\n")
    with open(os.path.join(d, "analysis", "plots", "grouping_summary.csv"), "w") as f:
        f.write("state_type,category,group_id,num_layers,layers,representative_layer,"
                "mean_similarity,min_similarity,max_similarity,notes\n")
        for st, cat, gid, layers, rep in groups:
            f.write(f'{st},{cat},{gid},{len(layers)},"{" ".join(map(str, layers))}",{rep},0.9,0.8,1.0,fixture\n')
    with open(os.path.join(d, "args.txt"), "w") as f:
        f.write(" ".join(args) + "\n")
    with tempfile.TemporaryDirectory() as tmp:
        work = os.path.join(tmp, "export")
        shutil.copytree(d, work)
        subprocess.run([CLI, work] + args, check=True, stdout=subprocess.DEVNULL)
        shutil.copytree(os.path.join(work, "prefix_mask_repair"), os.path.join(d, "expected"))


def main():
    if not os.path.exists(CLI):
        sys.exit("build oracle/_ref first: make -C oracle")
    rng = np.random.default_rng(2024)
    n = 1536

    # bf16 parameters, default masking (all 7 mantissa bits), two groups
    t = []
    for cat in ("q_proj", "mlp_up"):
        for layer in range(3):
            t.append(("param", cat, layer, "bfloat16", bf16(rng.standard_normal(n) * 0.02)))
    write_case("bf16_groups", t, [("param", "q_proj", 0, [0, 1, 2], 1), ("param", "mlp_up", 3, [0, 2], 2),
                                  ("param", "mlp_up", 4, [1], 1)], [])

    # fp32 Adam moments with partial masking and a rule cap
    t = [("exp_avg", "mlp_down", l, "float32", (rng.standard_normal(n) * 1e-3).astype(np.float32).view(np.uint32))
         for l in range(2)]
    t += [("exp_avg_sq", "mlp_down", l, "float32",
           ((rng.standard_normal(n) * 1e-3) ** 2 + 1e-12).astype(np.float32).view(np.uint32)) for l in range(2)]
    write_case("fp32_partial", t, [("exp_avg", "mlp_down", 0, [0, 1], 0), ("exp_avg_sq", "mlp_down", 1, [1, 0], 0)],
               ["--masked-mantissa-bits", "16", "--max-rules", "12"])

    # fp32 without masking: 32-bit symbols, mostly distinct (ties at low counts)
    base = (rng.standard_normal(64) * 1e-2).astype(np.float32).view(np.uint32)
    t = [("master", "attn_o", l, "float32", base[rng.integers(0, 64, 700)]) for l in range(2)]
    write_case("fp32_nomask", t, [("master", "attn_o", 0, [0, 1], 1)], ["--masked-mantissa-bits", "0"])

    # fp16 / fp16 alias: periodic sequences (many equal counts), constant runs,
    # and tensors of 0, 1, 2 and 3 elements
    per = np.tile(np.array([0x3C00, 0x4000, 0x3C00, 0x4200, 0xBC00], np.uint16), 40)
    t = [("param", "norm", 0, "float16", per),
         ("param", "norm", 1, "float16", np.full(301, 0x3C00, np.uint16)),
         ("param", "norm", 2, "float16", np.array([], np.uint16)),
         ("param", "norm", 3, "float16", np.array([0x3C00], np.uint16)),
         ("param", "norm", 4, "float16", np.array([0x3C00, 0x3C00], np.uint16)),
         ("param", "norm", 5, "float16", np.array([0x3C00, 0x3C00, 0x3C00], np.uint16)),
         ("param", "emb", 0, "fp16", (rng.standard_normal(900) * 0.5).astype(np.float16).view(np.uint16)),
         ("param", "emb", 1, "fp16", rng.integers(0, 1 << 16, 500).astype(np.uint16))]
    write_case("fp16_edge", t, [("param", "norm", 0, [0, 1, 2], 0), ("param", "norm", 1, [1, 3, 4, 5], 1),
                                ("param", "norm", 2, [2, 3], 3), ("param", "emb", 3, [0, 1], 0)],
               ["--masked-mantissa-bits", "6"])

    # filters select part of the grouping table; bf16 alias and short rule cap
    t = [(st, "gate", l, "bf16", bf16(rng.standard_normal(800) * s)) for st, s in (("param", 0.02), ("exp_avg", 1e-3))
         for l in range(2)]
    write_case("filtered", t, [("param", "gate", 0, [0, 1], 0), ("param", "gate", 1, [1], 1),
                               ("exp_avg", "gate", 0, [0, 1], 1)],
               ["--state-type", "param", "--category", "gate", "--group-id", "0", "--max-rules", "7"])


if __name__ == "__main__":
    main()
