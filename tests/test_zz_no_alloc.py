"""ckr_decode_noalloc (the decode that allocates nothing) against ckr_decode,
through the C ABI: bit-identical output and bad-lane counts on two calls in a
row on one GPU, the second with a smaller input, so the second call runs on the
scratch the first one left behind."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _case(ck, gpu, n, dt, unit, seed, corrupt=False):
    import torch
    g = torch.Generator(device=gpu).manual_seed(seed)
    if dt == ck.F32:
        t = torch.randn(n, device=gpu, generator=g) * 1e-3
    else:
        t = (torch.randn(n, device=gpu, generator=g) * 0.02).to(torch.bfloat16)
    enc = ck.compress(t.view(torch.uint8), dt, unit, n_elems=n)
    if corrupt:  # flip bytes in the middle of the coded data: some lanes must fail
        mid = enc.total // 2
        enc.data[mid:mid + 64] ^= 0x5A
    return t, enc


@pytest.mark.parametrize("first,second", [
    ((2_000_003, "F32", 65536, False), (70_001, "BF16", 65536, False)),
    ((1_500_000, "BF16", 1 << 20, True), (300_000, "F32", 1 << 20, False)),
    ((600_000, "F32", 0, False), (5_000, "F32", 4096, False)),
])
def test_decode_noalloc_matches_decode_on_two_calls(gpu, first, second):
    import torch
    import checkers_amd as ck
    outs = []
    for i, (n, dts, unit, corrupt) in enumerate((first, second)):
        dt = getattr(ck, dts)
        print(f"[case] noalloc call {i}: n={n} dtype={dts} unit={unit} corrupt={corrupt}", flush=True)
        t, enc = _case(ck, gpu, n, dt, unit, 100 + i, corrupt)
        nb = n * ck.element_size(dt)
        ref, bad_ref = ck.decode(enc)
        dst = torch.full((nb,), 0x77, dtype=torch.uint8, device=gpu)
        bad = ck.decode_noalloc(enc, dst)
        torch.cuda.synchronize()
        assert bad == bad_ref
        assert (bad > 0) == corrupt
        assert torch.equal(dst, ref[:nb])
        if not corrupt:
            assert torch.equal(dst, t.view(torch.uint8))
        outs.append(bad)


def test_decode_noalloc_refuses_what_it_cannot_do_without_allocating(gpu):
    import torch
    import checkers_amd as ck
    t, enc = _case(ck, gpu, 10_000, ck.BF16, 65536, 7)
    buf = torch.empty(20_000 + 8, dtype=torch.uint8, device=gpu)
    with pytest.raises(ck.CkrError) as e:   # a destination that is only element-aligned
        ck.decode_noalloc(enc, buf[2:2 + 20_000])
    assert e.value.code == ck.CKR_E_INVALID and "4-byte aligned" in str(e.value)
    torch.cuda.synchronize()


def test_decode_noalloc_captured_in_a_graph(gpu):
    """Captured into a HIP graph (h_bad_lanes NULL, as capture requires), the
    decode replays bit-exact, several times, with eager work between the
    replays; a capture that asks for the bad-lane count is refused; an eager
    call leaves the device's free memory unchanged."""
    import torch
    import checkers_amd as ck
    n = 1_000_003
    t, enc = _case(ck, gpu, n, ck.F32, 65536, 9)
    nb = n * 4
    ref, bad_ref = ck.decode(enc)
    assert bad_ref == 0
    dst = torch.zeros(nb, dtype=torch.uint8, device=gpu)
    assert ck.decode_noalloc(enc, dst) == 0          # warm-up: scratch address, code objects
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    assert ck.decode_noalloc(enc, dst) == 0
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0
    print("[case] noalloc decode under graph capture", flush=True)
    dst.zero_()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, capture_error_mode="relaxed"):
        with pytest.raises(ck.CkrError) as e:
            ck.decode_noalloc(enc, dst, check=True)
        ck.decode_noalloc(enc, dst, check=False)
    assert e.value.code == ck.CKR_E_INVALID and "captured" in str(e.value)
    torch.cuda.synchronize()
    assert not bool(dst.any())                        # capture ran nothing
    for r in range(4):
        dst.fill_(r + 1)                              # eager work between the replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(dst, ref[:nb]), r
    assert torch.equal(dst, t.view(torch.uint8))
    del g
