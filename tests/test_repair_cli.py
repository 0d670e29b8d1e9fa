"""The prefix-mask-repair command line (checkers_amd/ckr_prefix_mask_repair):
same arguments, reports and errors as the reference CLI.

GPU tests run it on every golden export directory and compare the three
reports with the reference CLI's, byte for byte except the time columns.
CPU tests cover the error paths that end before any device work.
"""
import os
import shutil
import subprocess

import pytest

from tests import repair_fixtures as rf

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "checkers_amd", "ckr_prefix_mask_repair")
REPORTS = ("tensor_prefix_mask_repair.csv", "group_prefix_mask_repair.csv",
           "checkpoint_prefix_mask_repair_summary.txt")


def run(args):
    return subprocess.run([CLI] + args, capture_output=True, text=True, timeout=120)


def copy_case(name, tmp_path):
    dst = tmp_path / name
    shutil.copytree(os.path.join(rf.GOLDEN, name), dst, ignore=shutil.ignore_patterns("expected"))
    return dst


def strip_time(text, fname):
    if not fname.endswith(".csv"):
        return text
    return "\n".join(",".join(line.split(",")[:-1]) for line in text.splitlines())


@pytest.mark.gpu
@pytest.mark.parametrize("name", rf.cases())
def test_cli_reports_match_reference(name, tmp_path):
    d = copy_case(name, tmp_path)
    args = open(os.path.join(d, "args.txt")).read().split()
    r = run([str(d)] + args)
    assert r.returncode == 0, r.stderr
    assert "Wrote tensor prefix-mask report to" in r.stdout
    for f in REPORTS:
        got = open(os.path.join(d, "prefix_mask_repair", f)).read()
        exp = open(os.path.join(rf.GOLDEN, name, "expected", f)).read()
        assert strip_time(got, f) == strip_time(exp, f), f


@pytest.mark.gpu
def test_cli_mixed_dtypes(tmp_path):
    d = copy_case("bf16_groups", tmp_path)
    m = open(os.path.join(d, "manifest.csv")).read().replace(",q_proj,param,1536,bfloat16,tensors/param_q_proj_2",
                                                              ",q_proj,param,1536,bf16,tensors/param_q_proj_2")
    open(os.path.join(d, "manifest.csv"), "w").write(m)
    r = run([str(d)])
    assert r.returncode == 1
    assert r.stderr.strip() == "tensor_group_prefix_mask_repair failed: Mixed dtypes inside one group are not supported"


@pytest.mark.parametrize("args,msg", [
    ([], "Usage: tensor_group_prefix_mask_repair <export_dir> [--state-type NAME] [--category NAME] "
         "[--group-id N] [--max-rules N] [--masked-mantissa-bits N]"),
    (["/nonexistent_dir"], "Failed to open manifest: /nonexistent_dir/manifest.csv"),
    (["@DIR", "--bogus", "1"], "Unknown or incomplete argument: --bogus"),
    (["@DIR", "--max-rules"], "Unknown or incomplete argument: --max-rules"),
    (["@DIR", "--state-type", "nothing"], "No matching grouping rows found for the requested filters"),
])
def test_cli_errors(args, msg, tmp_path):
    d = copy_case("bf16_groups", tmp_path)
    r = run([str(d) if a == "@DIR" else a for a in args])
    assert r.returncode == 1
    assert r.stderr.strip() == "tensor_group_prefix_mask_repair failed: " + msg


def test_cli_missing_representative_and_dtype(tmp_path):
    d = copy_case("bf16_groups", tmp_path)
    g = os.path.join(d, "analysis", "plots", "grouping_summary.csv")
    open(g, "a").write('param,q_proj,9,1,"7",7,0,0,0,x\n')
    r = run([str(d), "--group-id", "9"])
    assert r.returncode == 1
    assert r.stderr.strip().endswith("Missing representative tensor in manifest for requested group")
    m = os.path.join(d, "manifest.csv")
    open(m, "a").write("k,7,q_proj,param,4,int8,tensors/x.bin\n")
    r = run([str(d), "--group-id", "9"])
    assert r.stderr.strip().endswith("Unsupported dtype for mantissa-mask compression: int8")
