"""The `checkers_py` pybind11 module (checkers_api.cpp + python_bindings.cpp):
the reference module's surface (src/python_bindings.cpp:17-34), its error
behaviour (src/api.cpp:1028-1030, :1038-1040, :1262-1264, :1294-1297), the
discovery of src/api.cpp:416-887 against stand-in engines, and the files
compress_and_save writes, restored bit-exact through the reader."""
import re

import pytest

import checkers_amd as ck

checkers_py = pytest.importorskip("checkers_py", reason="checkers_py not built")


def test_module_surface():
    # exactly the reference's three functions, names, kwargs and defaults
    public = sorted(n for n in dir(checkers_py) if not n.startswith("_"))
    assert public == ["analyze_tensors", "compress_and_save", "initialize_context"]
    sig = checkers_py.initialize_context.__doc__.splitlines()[0]
    assert re.match(r"initialize_context\(model_engine: object, optimizer: object = None, "
                    r"histogram_bins: .*= 256, background_threads: .*= 1\) -> None", sig), sig
    assert checkers_py.analyze_tensors.__doc__.startswith("analyze_tensors() -> None")
    assert checkers_py.compress_and_save.__doc__.startswith("compress_and_save(arg0: str) -> None")
    with pytest.raises(TypeError):  # no py::arg in the reference: positional only
        checkers_py.compress_and_save(output_path="/tmp/x")


def test_errors_before_and_during_initialisation(capfd):
    # a context may already exist when GPU tests ran first in this process
    if checkers_py.__dict__.get("_initialised_here"):
        pytest.skip("context already created")
    with pytest.raises(RuntimeError, match=r"^\[checkers\] Context initialization failed: histogram_bins must be"):
        checkers_py.initialize_context(object(), histogram_bins=0)
    with pytest.raises(RuntimeError, match=r"^\[checkers\] Context initialization failed: background_threads must"):
        checkers_py.initialize_context(object(), background_threads=0)
    with pytest.raises(RuntimeError, match=r"^\[checkers\] Context initialization failed: .*module"):
        checkers_py.initialize_context(object())   # no .module
    with pytest.raises(RuntimeError, match=r"^Context not initialized: MemoryManager logger is null\.$"):
        checkers_py.analyze_tensors()
    with pytest.raises(RuntimeError, match=r"^Context not initialized: call initialize_context first\.$"):
        checkers_py.compress_and_save("/tmp/none")
    err = capfd.readouterr().err
    assert "[CHECKERS CRITICAL ERROR] Context not initialized" in err
    assert "[CHECKERS CRITICAL ERROR] compress_and_save: Context not initialized" in err


# ---- stand-ins for a DeepSpeed engine (only the attributes api.cpp reads)

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
    def __init__(self, named, opt=None, rank=0):
        self.module = _Module(named)
        self.optimizer = opt
        self.global_rank = rank


def _restore_all(tmp_path, rank, expected):
    """Restore every tensor of the rank's files; expected: name → source tensor."""
    import torch
    c = ck.Checkpoint(str(tmp_path), rank)
    names = [c.info(i)["name"] for i in range(len(c))]
    for i, name in enumerate(names):
        src = expected[name]
        out = c.restore(i)
        ref = src.contiguous().view(torch.uint8).reshape(-1)
        assert torch.equal(out[: ref.numel()], ref), name
    return names


@pytest.mark.gpu
@pytest.mark.parametrize("unit", ["65536", "0"])
def test_zero3_unaligned_offsets_round_trip(gpu, tmp_path, monkeypatch, unit):
    """Flat groups whose parameter offsets are not 16-byte multiples (odd
    element counts), parameters listed out of offset order, one parameter
    outside this rank's territory; every tracked tensor restores bit-exact."""
    import torch
    checkers_py._initialised_here = True
    monkeypatch.setenv("CHECKERS_UNIT_BYTES", unit)
    g = torch.Generator(device=gpu).manual_seed(3)
    sizes = [[5001, 3003, 70001], [4097]]
    named, pos, flat16, flat32, state, src = [], {}, [], [], {}, {}
    for gi, sz in enumerate(sizes):
        total = sum(sz)
        f32 = torch.randn(total, device=gpu, generator=g) * 0.02
        flat32.append(f32)
        flat16.append(f32.to(torch.bfloat16))
        ea = torch.randn(total, device=gpu, generator=g) * 1e-3
        easq = torch.randn(total, device=gpu, generator=g) ** 2 * 1e-6 + 1e-12
        state[f32] = {"exp_avg": ea, "exp_avg_sq": easq}
        off = 0
        for pi, n in enumerate(sz):
            p = _Param(n)
            pos[id(p)] = [gi, off, n]
            pn = f"layers.{gi}.w{pi}"
            named.append((pn, p))
            src[pn] = flat16[-1][off:off + n]
            src["master_weights::" + pn] = f32[off:off + n]
            src["optimizer.exp_avg::" + pn] = ea[off:off + n]
            src["optimizer.exp_avg_sq::" + pn] = easq[off:off + n]
            off += n
    named.reverse()
    eng = _Engine(named, _ZeroOpt(flat16, flat32, state, pos))
    checkers_py.initialize_context(eng)
    checkers_py.analyze_tensors()
    checkers_py.compress_and_save(str(tmp_path))
    names = _restore_all(tmp_path, 0, src)
    exp = []
    for pn in ("layers.0.w0", "layers.0.w1", "layers.0.w2", "layers.1.w0"):   # flat-offset order
        exp += [pn, "master_weights::" + pn, "optimizer.exp_avg::" + pn, "optimizer.exp_avg_sq::" + pn]
    assert names == exp
    c = ck.Checkpoint(str(tmp_path), 0)
    # bfloat16 carries the float16 tag (parse_dtype's order of tests, api.cpp:887-893)
    assert [c.info(i)["dtype"] for i in range(4)] == [ck.F16, ck.F32, ck.F32, ck.F32]
    assert sum(c.info(i)["owns_table"] for i in range(len(c))) <= len(c)


@pytest.mark.gpu
def test_plain_parameters_partitions_gather_and_host_skip(gpu, tmp_path, monkeypatch):
    """The non-ZeRO-3 path: plain parameters, a ds_tensor partition of rank 1,
    a non-contiguous (transposed) parameter gathered into the arena, a host
    tensor skipped; compress without analyze makes every tensor a singleton."""
    import torch
    checkers_py._initialised_here = True
    monkeypatch.setenv("CHECKERS_UNIT_BYTES", "4096")
    torch.manual_seed(0)
    lin = torch.nn.Linear(64, 130).to(gpu)
    wt = torch.nn.Parameter(torch.randn(96, 40, device=gpu).t())          # strides (1, 40)
    assert not wt.is_contiguous()
    host = torch.nn.Parameter(torch.randn(8))
    part = _Param(1000)
    part.ds_tensor = torch.randn(600, device=gpu)                           # rank 1 holds 400 of them
    part.partition_numel = lambda: 600
    named = [("lin.weight", lin.weight), ("lin.bias", lin.bias), ("wt", wt), ("host", host), ("part", part)]
    checkers_py.initialize_context(_Engine(named, rank=1))
    checkers_py.compress_and_save(str(tmp_path))
    src = {"lin.weight": lin.weight.detach(), "lin.bias": lin.bias.detach(), "wt": wt.detach(),
           "part": part.ds_tensor[:400]}
    names = _restore_all(tmp_path, 1, src)
    assert names == ["lin.weight", "lin.bias", "wt", "part"]
    c = ck.Checkpoint(str(tmp_path), 1)
    assert all(c.info(i)["owns_table"] == 1 for i in range(len(c)))
    assert c.info(3)["num_elements"] == 400
