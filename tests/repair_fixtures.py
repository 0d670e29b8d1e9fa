"""Readers for the prefix-mask-repair golden fixtures (tests/golden/repair/)."""
import csv
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "repair")
LAYOUT = {"float32": (4, 23), "float16": (2, 10), "fp16": (2, 10), "bfloat16": (2, 7), "bf16": (2, 7)}


def cases():
    return sorted(d for d in os.listdir(GOLDEN) if os.path.isdir(os.path.join(GOLDEN, d)))


def load_case(name):
    d = os.path.join(GOLDEN, name)
    with open(os.path.join(d, "args.txt")) as f:
        args = f.read().split()
    opts = dict(max_rules=50, masked=None, state_type=None, category=None, group_id=None)
    it = iter(args)
    for a in it:
        v = next(it)
        if a == "--max-rules":
            opts["max_rules"] = int(v)
        elif a == "--masked-mantissa-bits":
            opts["masked"] = int(v)
        elif a == "--state-type":
            opts["state_type"] = v
        elif a == "--category":
            opts["category"] = v
        elif a == "--group-id":
            opts["group_id"] = int(v)
    manifest = {}
    with open(os.path.join(d, "manifest.csv")) as f:
        for row in list(csv.reader(f))[1:]:
            key, layer, cat, st, numel, dt, fn = row
            es = LAYOUT[dt][0]
            raw = np.fromfile(os.path.join(d, fn), np.uint8)
            assert raw.size == int(numel) * es
            manifest[(st, cat, int(layer))] = dict(numel=int(numel), dtype=dt, raw=raw)
    groups = []
    with open(os.path.join(d, "analysis", "plots", "grouping_summary.csv")) as f:
        for row in list(csv.reader(f))[1:]:
            st, cat, gid, _, layers, rep = row[:6]
            if opts["state_type"] and st != opts["state_type"]:
                continue
            if opts["category"] and cat != opts["category"]:
                continue
            if opts["group_id"] is not None and int(gid) != opts["group_id"]:
                continue
            groups.append(dict(state_type=st, category=cat, group_id=int(gid),
                               layers=[int(x) for x in layers.split()], rep=int(rep)))

    def rows(fn):
        with open(os.path.join(d, "expected", fn)) as f:
            r = list(csv.reader(f))
        return r[0], r[1:]

    return dict(dir=d, args=args, opts=opts, manifest=manifest, groups=groups,
                tensor_rows=rows("tensor_prefix_mask_repair.csv"),
                group_rows=rows("group_prefix_mask_repair.csv"))


def bit_width(count):
    """bit_width_for_symbol_count (tensor_group_prefix_mask_repair.cpp:204-217)."""
    return max(1, (count - 1).bit_length()) if count > 1 else 1


def evaluate(case, build, apply_):
    """Per-tensor (token_count, rule_count, payload, grammar, residual, masked_only)
    and per-group (rule_count, max_pair) through the given build/apply callables:
    build(raw, n, es, masked_bits, max_rules) -> dict(rules, out_len, max_pair);
    apply_(raw, n, es, masked_bits, rules) -> token count."""
    out_t, out_g = [], []
    for g in case["groups"]:
        rep = case["manifest"][(g["state_type"], g["category"], g["rep"])]
        es, mb = LAYOUT[rep["dtype"]]
        k = mb if case["opts"]["masked"] is None else min(case["opts"]["masked"], mb)
        gr = build(rep["raw"], rep["numel"], es, k, case["opts"]["max_rules"])
        nr = len(gr["rules"])
        width = bit_width((1 << (8 * es - k)) + nr)
        grammar = (width * 2 * nr + 7) // 8
        charged = False
        for layer in g["layers"]:
            t = case["manifest"][(g["state_type"], g["category"], layer)]
            tok = gr["out_len"] if layer == g["rep"] else apply_(t["raw"], t["numel"], es, k, gr["rules"])
            payload = (width * tok + 7) // 8
            out_t.append(dict(layer=layer, tokens=tok, rules=nr, payload=payload,
                              grammar=0 if charged else grammar,
                              residual=(t["numel"] * k + 7) // 8,
                              masked_only=(t["numel"] * (8 * es - k) + 7) // 8,
                              original=t["numel"] * es, masked_bits=k))
            charged = True
        out_g.append(dict(rules=nr, max_pair=gr["max_pair"], grammar=grammar))
    return out_t, out_g
