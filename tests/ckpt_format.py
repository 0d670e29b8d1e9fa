"""The .ansc v4 unit records restated in Python, independently of the C++
writer and reader: pack (headers + unit data → record + stored bytes) and
expand (the inverse).  Tests compare the library's files with pack() applied to
the oracle's streams, and build files for the reader's checks with it.

Unit record by kind (first byte): 1 raw (bytes stored as they are); 0 packed
(per live plane u32 base + u8 width, then an LSB-first bit stream of the live
lanes' 31-bit final states and their count - base deltas; stored bytes: live
lanes only); 2 full (256 x (u32 state, u32 count), every lane's bytes)."""
import struct

import numpy as np

L = 1 << 23
HEADER = np.dtype([("final_state", "<u4"), ("byte_count", "<u4"), ("buf_offset", "<u4"), ("pad", "<u4")])


def zero_lane(norm0, K):
    """(final state, bytes in stored order) of K zero symbols encoded with
    frequency norm0 (0: each symbol a raw byte)."""
    x, rev = L, []
    for _ in range(K):
        if norm0 == 0:
            rev.append(0)
            continue
        while x >= norm0 << 19:
            rev.append(x & 255)
            x >>= 8
        x = ((x // norm0) << 12) + (x % norm0)
    return x, bytes(reversed(rev))


def _lane_k(length):
    t = np.arange(256)
    return np.where(length > t, (length - t + 255) // 256, 0)


def pack_unit(h, unit_data, length, es, spe, norm0):
    """(record, stored bytes) of one unit: h its 256 headers, unit_data its bytes."""
    cnt = h["byte_count"].astype(np.int64)
    st = h["final_state"].astype(np.int64)
    if length > 0 and cnt[0] == length and cnt[1:].sum() == 0:
        return b"\x01", bytes(unit_data[:length])
    t = np.arange(256)
    live = (t % es) >= spe
    K = _lane_k(length)
    odd = bool((st[live] >= 1 << 31).any())
    for lane in np.nonzero(~live)[0]:
        zs, zb = zero_lane(norm0, int(K[lane]))
        odd = odd or (zs, len(zb)) != (int(st[lane]), int(cnt[lane]))
    if odd:
        rec = b"\x02" + b"".join(struct.pack("<II", int(st[i]), int(cnt[i])) for i in range(256))
        return rec, bytes(unit_data[: int(cnt.sum())])
    G = es - spe
    base, w = [], []
    for g in range(G):
        c = cnt[t % es == spe + g]
        base.append(int(c.min()))
        w.append(int(c.max() - c.min()).bit_length())
    lanes = np.nonzero(live)[0]
    acc, pos = 0, 0
    for lane in lanes:
        acc |= int(st[lane]) << pos
        pos += 31
    for lane in lanes:
        g = lane % es - spe
        acc |= (int(cnt[lane]) - base[g]) << pos
        pos += w[g]
    rec = b"\x00" + b"".join(struct.pack("<IB", base[g], w[g]) for g in range(G)) + acc.to_bytes((pos + 7) // 8,
                                                                                                "little")
    stored = b"".join(bytes(unit_data[int(h[lane]["buf_offset"]): int(h[lane]["buf_offset"]) + int(cnt[lane])])
                      for lane in lanes)
    return rec, stored


def pack_tensor(headers, unit_offsets, data, n_bytes, unit, es, spe, norm0):
    """Records and stored bytes of a tensor encoded in units of `unit` bytes."""
    unit = min(unit, n_bytes)
    nu = (n_bytes + unit - 1) // unit
    recs, stored = [], []
    for u in range(nu):
        length = min(unit, n_bytes - u * unit)
        ud = data[int(unit_offsets[u]): int(unit_offsets[u + 1])]
        r, s = pack_unit(headers[u * 256:(u + 1) * 256], ud, length, es, spe, norm0)
        recs.append(r)
        stored.append(s)
    return b"".join(recs), b"".join(stored)


def expand_tensor(rec, stored, n_bytes, unit, es, spe, norm0):
    """(headers, unit offsets, data) from records and stored bytes."""
    unit = min(unit, n_bytes)
    nu = (n_bytes + unit - 1) // unit
    hdr = np.zeros(nu * 256, HEADER)
    uoff = np.zeros(nu + 1, np.uint64)
    out, rp, sp = [], 0, 0
    t = np.arange(256)
    live = (t % es) >= spe
    for u in range(nu):
        length = min(unit, n_bytes - u * unit)
        h = hdr[u * 256:(u + 1) * 256]
        kind = rec[rp]
        if kind == 1:
            rp += 1
            h[0]["byte_count"] = length
            out.append(stored[sp: sp + length])
            sp += length
            uoff[u + 1] = uoff[u] + length
            continue
        if kind == 2:
            vals = np.frombuffer(rec, "<u4", 512, rp + 1).reshape(256, 2)
            rp += 1 + 2048
            h["final_state"], h["byte_count"] = vals[:, 0], vals[:, 1]
            body = stored[sp: sp + int(vals[:, 1].sum())]
            sp += len(body)
        else:
            G = es - spe
            base = [struct.unpack_from("<I", rec, rp + 1 + 5 * g)[0] for g in range(G)]
            w = [rec[rp + 5 + 5 * g] for g in range(G)]
            lanes = np.nonzero(live)[0]
            nbits = 31 * len(lanes) + (256 // es) * sum(w)
            bs = rp + 1 + 5 * G
            acc = int.from_bytes(rec[bs: bs + (nbits + 7) // 8], "little")
            rp = bs + (nbits + 7) // 8
            pos = 0
            for lane in lanes:
                h[lane]["final_state"] = (acc >> pos) & 0x7FFFFFFF
                pos += 31
            for lane in lanes:
                g = lane % es - spe
                h[lane]["byte_count"] = base[g] + ((acc >> pos) & ((1 << w[g]) - 1))
                pos += w[g]
            K = _lane_k(length)
            parts = []
            for lane in range(256):
                if live[lane]:
                    c = int(h[lane]["byte_count"])
                    parts.append(stored[sp: sp + c])
                    sp += c
                else:
                    zs, zb = zero_lane(norm0, int(K[lane]))
                    h[lane]["final_state"], h[lane]["byte_count"] = zs, len(zb)
                    parts.append(zb)
            body = b"".join(parts)
        h["buf_offset"] = np.concatenate([[0], np.cumsum(h["byte_count"].astype(np.int64))[:-1]])
        out.append(body)
        uoff[u + 1] = uoff[u] + len(body)
    assert rp == len(rec) and sp == len(stored)
    return hdr, uoff, b"".join(out)
