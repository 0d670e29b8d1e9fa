"""The table built on the device (ckr_build_tables_device: one workgroup per
histogram, one thread per symbol) against the host's: 10^5 histograms of the
seven families of test_table_ranked, every row equal to the host's ranked
table (counts, sum, ambiguity flag) and, where not ambiguous, to the sorted
table of the reference's normalize_histogram (src/ANSCompressor.cpp:416-503).
Then ckr_compress through its device-table path on a tensor whose table is
ambiguous: the host's sorted table takes over, bytes equal to the oracle's."""
import numpy as np
import pytest

import oracle as oc
from tests import datagen as dg
from tests.test_table_ranked import histograms

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("ensure", [False, True])
def test_device_tables_equal_host_tables(ensure, gpu):
    import torch
    import checkers_amd as ck
    hs = histograms(11 + int(ensure), 50_000)
    print(f"[case] {len(hs)} device tables ensure_full={ensure}", flush=True)
    rows = ck.build_tables_device(torch.from_numpy(hs.view(np.int32)).to(gpu), ensure)
    torch.cuda.synchronize()
    rows = rows.cpu().numpy().view(np.uint32)
    n_amb = 0
    for i, h in enumerate(hs):
        got, amb = ck.build_table_ranked(h, ensure)
        assert np.array_equal(rows[i, :256], got.norm), (i, h)
        assert rows[i, 256] == int(got.norm.sum()) and rows[i, 257] == int(amb), i
        if amb:
            n_amb += 1
            continue
        ref, _ = ck.build_table(h, ensure)
        assert np.array_equal(rows[i, :256], ref.norm), (i, h)
    assert n_amb > 0


def test_compress_with_an_ambiguous_device_table(gpu):
    """bf16 values whose high bytes take three values 1000 times each: the three
    fractional parts are equal and two of the three symbols get the last two
    slots, which only the reference's sort decides."""
    import torch
    import checkers_amd as ck
    hi = np.repeat(np.array([0x3F, 0x40, 0xBF], np.uint16), 1000)
    raw = ((hi << 8) | np.arange(3000, dtype=np.uint16) % 256).astype(np.uint16)
    h = np.zeros(256, np.uint32)
    h[0], h[0x3F], h[0x40], h[0xBF] = 3000, 1000, 1000, 1000   # the masked histogram
    assert ck.build_table_ranked(h, False)[1]
    ref = oc.compress_tensor(raw, raw.size, dg.BF16, 65536)
    src = torch.from_numpy(raw.view(np.int16).copy()).to(gpu)
    enc = ck.compress(src.view(torch.uint8), dg.BF16, 65536, n_elems=raw.size)
    torch.cuda.synchronize()
    assert np.array_equal(enc.table.norm, ref["table"]["norm_freq"])
    assert enc.total == ref["data"].size and np.array_equal(enc.data_np(), ref["data"])
    dst, bad = ck.decode(enc)
    torch.cuda.synchronize()
    assert bad == 0 and np.array_equal(dst.cpu().numpy(), raw.view(np.uint8))
