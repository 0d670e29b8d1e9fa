"""Rank checkpoint files at the configurations' sizes, written and restored.

- cfg3 through the drop-in: checkers_py.initialize_context / analyze_tensors /
  compress_and_save on a stand-in ZeRO-3 engine over the full Llama-3-8B
  rank-0-of-8 shard (4 x 1,003,782,656 elements, 14.05 GB, .ansc v4 with 64 KiB
  units), then every tensor restored from the files bit-exact.  Each tensor's
  stored bytes span 14 to 60 of the writer's 32 MiB staging chunks.
- One fp32 tensor above 4 GiB (the case the reference's u32 header fields
  cannot hold, include/checkers/ANSCompressor.hpp:79-84) written as v4 and
  restored; at the default 4 GiB slice it is encoded in two slices.
- One fp32 tensor just below 2^32 bytes written as v2 (the reference's own
  single-stream layout, src/ANSCompressor.cpp:721-816) and restored.
- The writer's device buffers: slices of whole units give the same files as
  whole tensors, and the buffers do not grow with the tensors.
"""
import os
import types

import numpy as np
import pytest

from tests import datagen as dg

pytestmark = pytest.mark.gpu


def _ck():
    import checkers_amd as ck
    return ck


def _gen(gpu, seed):
    import torch
    return torch.Generator(device=gpu).manual_seed(seed)


class _ZeroParam:
    """A ZeRO-3 parameter as api.cpp reads it: requires_grad and ds_numel."""

    def __init__(self, n):
        self.requires_grad = True
        self.ds_numel = n


def _zero3_engine(params, master, exp_avg, exp_avg_sq):
    """One ZeRO-3 flat group holding the shard: fp16 flat = params, fp32 flat =
    master, optimizer state = exp_avg and exp_avg_sq (src/api.cpp:416-685)."""
    n = master.numel()
    p = _ZeroParam(n)
    opt = types.SimpleNamespace(
        fp16_partitioned_groups_flat=[params], fp32_partitioned_groups_flat=[master],
        optimizer=types.SimpleNamespace(state={master: {"exp_avg": exp_avg, "exp_avg_sq": exp_avg_sq}}),
        grad_position={id(p): [0, 0, n]}, get_param_id=id)
    return types.SimpleNamespace(module=types.SimpleNamespace(named_parameters=lambda: iter([("layers.flat", p)])),
                                 optimizer=opt, global_rank=0)


def _restore_equal(c, i, src):
    import torch
    ref = src.contiguous().view(torch.uint8).reshape(-1)
    out = c.restore(i)
    ok = torch.equal(out[: ref.numel()], ref)
    del out
    torch.cuda.empty_cache()
    return ok


def test_cfg3_compress_and_save_restores_every_tensor(gpu, tmp_path, monkeypatch):
    import torch
    import checkers_py
    ck = _ck()
    checkers_py._initialised_here = True
    monkeypatch.setenv("CHECKERS_UNIT_BYTES", "65536")
    n = 1_003_782_656
    g = _gen(gpu, 31)
    print("[case] cfg3 shard through checkers_py.compress_and_save, then restore", flush=True)
    params = (torch.randn(n, device=gpu, generator=g) * 0.02).to(torch.bfloat16)
    master = params.float()
    exp_avg = torch.randn(n, device=gpu, generator=g) * 1e-3
    exp_avg_sq = torch.randn(n, device=gpu, generator=g).mul_(1e-3)
    exp_avg_sq.mul_(exp_avg_sq).add_(1e-12)
    checkers_py.initialize_context(_zero3_engine(params, master, exp_avg, exp_avg_sq))
    checkers_py.analyze_tensors()
    # the writer's buffers were reserved by initialize_context: two sets of
    # {packed, stored, sidecar, headers, records} for one slice (each tensor is
    # one slice here) and the encode workspace, not the shard's 14 GB
    reserved = ck.ckpt_pool_bytes()
    assert 0 < reserved < 6 * 4.1e9
    checkers_py.compress_and_save(str(tmp_path))
    assert ck.ckpt_pool_bytes() == reserved
    c = ck.Checkpoint(str(tmp_path), 0)
    names = [c.info(i)["name"] for i in range(len(c))]
    assert names == ["layers.flat", "master_weights::layers.flat", "optimizer.exp_avg::layers.flat",
                     "optimizer.exp_avg_sq::layers.flat"]
    for i, src in enumerate((params, master, exp_avg, exp_avg_sq)):
        info = c.info(i)
        assert info["version"] == 4 and info["num_elements"] == n
        # more than ten 32 MiB staging chunks per tensor went through the ring
        assert info["data_size"] > 10 * (32 << 20)
        print(f"[case] cfg3 restore {names[i]}", flush=True)
        assert _restore_equal(c, i, src), names[i]
    c.close()


def test_fp32_tensor_above_4gib_v4_two_slices(gpu, tmp_path):
    """1.1e9 fp32 elements (4.4 GB): v4 files, two slices at the default 4 GiB
    slice size, restored bit-exact."""
    import torch
    ck = _ck()
    n = 1_100_000_001
    print("[case] fp32 tensor of 4.4 GB, v4, 64 KiB units", flush=True)
    x = torch.randn(n, device=gpu, generator=_gen(gpu, 41)) * 1e-3
    assert n * 4 > (1 << 32)
    try:
        stats = ck.write_checkpoint(str(tmp_path), 0, [("big", x.view(torch.uint8), ck.F32, -1)], unit_bytes=65536)
        assert stats[0]["n_slices"] == 2 and stats[0]["original_bytes"] == n * 4
        c = ck.Checkpoint(str(tmp_path), 0)
        info = c.info(0)
        assert info["version"] == 4 and info["num_elements"] == n and info["n_units"] == -(-n * 4 // 65536)
        assert _restore_equal(c, 0, x)
        c.close()
    finally:
        ck.release_checkpoint_buffers()


def test_fp32_tensor_just_below_4gib_v2(gpu, tmp_path):
    """The reference's single-stream layout at its limit: 2^32 - 256 bytes of
    fp32 in one stream of 256 lanes (u32 byte counts and offsets), restored."""
    import torch
    ck = _ck()
    n = ((1 << 32) - 256) // 4
    print("[case] fp32 tensor of 2^32-256 bytes, v2 (one stream)", flush=True)
    x = torch.randn(n, device=gpu, generator=_gen(gpu, 43)) * 1e-3
    try:
        stats = ck.write_checkpoint(str(tmp_path), 0, [("w", x.view(torch.uint8), ck.F32, -1)], unit_bytes=0)
        assert stats[0]["n_slices"] == 1
        c = ck.Checkpoint(str(tmp_path), 0)
        info = c.info(0)
        assert info["version"] == 2 and info["n_units"] == 1 and info["original_bytes"] == n * 4
        assert _restore_equal(c, 0, x)
        c.close()
    finally:
        ck.release_checkpoint_buffers()


def _files(d, rank):
    return [open(os.path.join(d, p), "rb").read() for p in
            (f"rank_{rank}_states.ansc", f"mantissa/rank_{rank}_mantissa.mant", f"tables/rank_{rank}_tables.dict")]


@pytest.mark.parametrize("unit", [65536, 4096])
def test_slices_give_the_same_files_and_bounded_buffers(gpu, tmp_path, unit):
    """Tensors of many units written in slices of three units give, byte for
    byte, the files they give written whole (clusters, raw units and ragged last
    units included); with the slice size fixed, tensors four times larger leave
    the writer's device buffers where they were; every tensor restores."""
    import torch
    ck = _ck()

    def recs(scale, seed):
        rng = np.random.default_rng(seed)
        m = unit // 4 * scale
        bf = dg.normal_bf16(7 * m + 1001, 0.02, seed + 1)
        return [("layers.0.w", bf, dg.BF16, 0),
                ("layers.1.w", dg.normal_bf16(5 * m + 77, 0.02, seed + 2), dg.BF16, 0),
                ("master_weights::layers.0.w", (bf.astype(np.uint32) << 16).view(np.float32), dg.F32, -1),
                ("optimizer.exp_avg::layers.0.w", dg.normal_f32(9 * m + 3, 1e-3, seed + 3), dg.F32, -1),
                ("optimizer.exp_avg_sq::layers.0.w", dg.exp_avg_sq(6 * m + 5, seed + 4), dg.F32, -1),
                ("noise", rng.integers(0, 256, 4 * unit * scale + 9).astype(np.uint8).view(np.int8), dg.I8, -1)]

    def dev(recs_):
        out = []
        for name, arr, tag, cid in recs_:
            b = np.ascontiguousarray(arr).view(np.uint8).reshape(-1)
            out.append((name, torch.from_numpy(b.copy()).to(gpu), tag, cid))
        return out

    small = dev(recs(1, 3))
    try:
        ck.release_checkpoint_buffers()
        ck.set_ckpt_slice_bytes(1 << 40)          # one slice per tensor
        whole = ck.write_checkpoint(str(tmp_path / "whole"), 2, small, unit_bytes=unit, repair_tables=True)
        assert all(s["n_slices"] == 1 for s in whole)
        ck.release_checkpoint_buffers()
        ck.set_ckpt_slice_bytes(3 * unit)
        sliced = ck.write_checkpoint(str(tmp_path / "sliced"), 2, small, unit_bytes=unit, repair_tables=True)
        assert sum(s["n_slices"] >= 2 for s in sliced) == 5     # all but the 2.5-unit layers.1.w
        for a, b in zip(whole, sliced):
            for k in ("ans_bytes", "stored_bytes", "record_bytes", "sidecar_bytes", "table_sum", "owns_table"):
                assert a[k] == b[k], k
        for a, b, what in zip(_files(tmp_path / "whole", 2), _files(tmp_path / "sliced", 2), ("ansc", "mant", "dict")):
            assert a == b, what
        held = ck.ckpt_pool_bytes()
        large = dev(recs(4, 5))
        stats = ck.write_checkpoint(str(tmp_path / "large"), 2, large, unit_bytes=unit, repair_tables=True)
        assert max(s["n_slices"] for s in stats) >= 8
        assert ck.ckpt_pool_bytes() == held
        c = ck.Checkpoint(str(tmp_path / "large"), 2)
        for i, (name, t, tag, cid) in enumerate(large):
            assert torch.equal(c.restore(i)[: t.numel()], t), name
        c.close()
    finally:
        ck.set_ckpt_slice_bytes(0)
        ck.release_checkpoint_buffers()
