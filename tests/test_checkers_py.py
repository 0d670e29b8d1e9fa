"""The checkers_py drop-in surface: discovery order and names, dtype tags,
error wrapping, and the files compress_and_save writes (restored bit-exact)."""
import numpy as np
import pytest

import checkers_amd as ck
from checkers_amd import checkers_py as cp


def test_dtype_parse_quirk_and_errors(capsys):
    # bfloat16 contains "float16": the reference tags it float16 (api.cpp:887-893)
    assert cp._parse_dtype("torch.bfloat16") == ck.F16
    assert cp._parse_dtype("torch.float32") == ck.F32 and cp._parse_dtype("torch.float16") == ck.F16
    assert cp._parse_dtype("torch.int8") == ck.I8 and cp._parse_dtype("torch.int32") == ck.UNKNOWN
    with pytest.raises(RuntimeError, match=r"^\[checkers\] Context initialization failed: histogram_bins"):
        cp.initialize_context(object(), histogram_bins=0)
    with pytest.raises(RuntimeError, match="background_threads must be greater than zero"):
        cp.initialize_context(object(), background_threads=0)
    cp._ctx = None
    with pytest.raises(RuntimeError, match="Context not initialized"):
        cp.compress_and_save("/tmp/none")
    assert "[CHECKERS CRITICAL ERROR] compress_and_save:" in capsys.readouterr().err


class _Param:
    def __init__(self, ds_numel):
        self.requires_grad = True
        self.ds_numel = ds_numel


class _Base:
    def __init__(self, state):
        self.state = state


class _ZeroOpt:
    def __init__(self, fp16, fp32, state, positions):
        self.fp16_partitioned_groups_flat = fp16
        self.fp32_partitioned_groups_flat = fp32
        self.optimizer = _Base(state)
        self.grad_position = positions

    def get_param_id(self, p):
        return id(p)


class _Module:
    def __init__(self, named):
        self._named = named

    def named_parameters(self):
        return iter(self._named)


class _Engine:
    def __init__(self, named, opt, rank=0):
        self.module = _Module(named)
        self.optimizer = opt
        self.global_rank = rank


@pytest.mark.gpu
def test_zero3_discovery_and_round_trip(gpu, tmp_path):
    import torch
    g = torch.Generator(device=gpu).manual_seed(3)
    # two flat groups; parameters listed out of offset order; one parameter
    # beyond this rank's slice (skipped)
    sizes = [[5000, 3000], [4000]]
    named, pos, flat16, flat32, state = [], {}, [], [], {}
    for gi, sz in enumerate(sizes):
        total = sum(sz)
        f32 = torch.randn(total, device=gpu, generator=g) * 0.02
        flat32.append(f32)
        flat16.append(f32.to(torch.bfloat16))
        state[f32] = {"exp_avg": torch.randn(total, device=gpu, generator=g) * 1e-3,
                      "exp_avg_sq": torch.randn(total, device=gpu, generator=g) ** 2 * 1e-6 + 1e-12}
        off = 0
        for pi, n in enumerate(sz):
            p = _Param(n)
            pos[id(p)] = [gi, off, n]
            named.append((f"layers.{gi}.w{pi}", p))
            off += n
    extra = _Param(7)
    named.append(("beyond", extra))
    pos[id(extra)] = [1, 4000, 0]       # no resident elements: not tracked
    named.reverse()
    eng = _Engine(named, _ZeroOpt(flat16, flat32, state, pos))
    cp.initialize_context(eng)
    names = [r[0] for r in cp.records()]
    exp = []
    for pn in ("layers.0.w0", "layers.0.w1", "layers.1.w0"):
        exp += [pn, "master_weights::" + pn, "optimizer.exp_avg::" + pn, "optimizer.exp_avg_sq::" + pn]
    assert names == exp
    assert [r[1] for r in cp.records()][:2] == [ck.F16, ck.F32]   # bf16 tagged float16
    cp.analyze_tensors()
    assert len(cp._ctx.cluster_of) == len(exp)
    cp.compress_and_save(str(tmp_path))
    c = ck.Checkpoint(str(tmp_path), 0)
    assert [c.info(i)["name"] for i in range(len(c))] == exp
    srcs = {r.name: r.tensor for r in cp._ctx.records}
    restored = 0
    for i in range(len(c)):
        info = c.info(i)
        assert info["dtype"] == (ck.F16 if "::" not in info["name"] else ck.F32)
        try:
            out = c.restore(i)
        except ck.CkrError as e:
            # only a cluster table the reference's normalisation left above 4096
            assert e.code == ck.CKR_E_TABLE and "not 4096" in str(e)
            continue
        t = srcs[info["name"]]
        assert torch.equal(out[: t.numel() * t.element_size()], t.view(torch.uint8).reshape(-1))
        restored += 1
    assert restored >= len(exp) // 2


@pytest.mark.gpu
def test_plain_parameters_round_trip(gpu, tmp_path):
    import torch
    torch.manual_seed(0)
    m = torch.nn.Sequential(torch.nn.Linear(64, 128), torch.nn.Linear(128, 16)).to(gpu)

    class Eng:
        module = m
        optimizer = None
        global_rank = 2

    cp.initialize_context(Eng())
    assert [r[0] for r in cp.records()] == ["0.weight", "0.bias", "1.weight", "1.bias"]
    cp.compress_and_save(str(tmp_path), unit_bytes=4096)   # no analyze: all singletons
    c = ck.Checkpoint(str(tmp_path), 2)
    for i, (name, p) in enumerate(m.named_parameters()):
        assert c.info(i)["name"] == name and c.info(i)["owns_table"] == 1
        out = c.restore(i)
        assert torch.equal(out[: p.numel() * 4], p.detach().view(torch.uint8).reshape(-1))
