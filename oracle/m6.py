"""ORACLE -- test infrastructure only. Never imported by the product (seedpack_amd/).

CPU restatement of the reference's M6 codec model (seedpack/gpu_codec.py, cited as gpu_codec.py:LINES)
as its --cpu path computes it: per tensor the median of the scale bits and 16 column classes by the
quantiles of the column RMS (gpu_codec.py:229-236), each block's largest-|weight| position
(gpu_codec.py:238), the symbols of each segment of 512 blocks with their tables (gpu_codec.py:63-77),
the table normalisation (gpu_codec.py:193-209) and a textbook rANS coder per segment (PB 12, RANS_L
2^23, byte renormalisation, the state's 4 bytes last written; gpu_codec.py:95-157).

Pinned by tests/test_oracle_m6.py against tests/golden/m6_vectors.npz (the reference's own M6GPU run
through its --cpu backend, tests/golden/make_m6_golden.py): medians, column classes, tables, segment
lengths and stream; by round trips; and by a planted mistake (the hi context not reset at a segment's
first block).
"""
import numpy as np

SEG, PB, N_COL, N_SB = 512, 12, 16, 16
TPG = 256 + 256 + 1 + 1 + N_SB * N_COL
T_HI, T_LO, T_POS, T_MX, T_QS = 0, 256, 512, 513, 514
RANS_L = 1 << 23


def stats(blocks, layout):
    """-> (med per tensor, colmap over all tensors' columns)"""
    med, cms, f = [], [], 0
    for _, nbytes, rowlen, _ in layout["t"]:
        nb = nbytes // 34
        b = blocks[f:f + nb]
        bits = b[:, 0].astype(np.int32) | (b[:, 1].astype(np.int32) << 8)
        med.append(int(np.median(bits)))
        q = b[:, 2:].view(np.int8).reshape(-1, rowlen).astype(np.float32)
        rms = np.sqrt((q * q).mean(0))
        edges = np.quantile(rms, np.linspace(0, 1, N_COL + 1)[1:-1])
        cms.append(np.searchsorted(edges, rms).astype(np.uint8))
        f += nb
    return med, np.concatenate(cms)


def meta_of(layout, med):
    groups = sorted({t[3] for t in layout["t"]})
    rows, first, colbase = [], 0, 0
    for i, (_, nbytes, rowlen, grp) in enumerate(layout["t"]):
        nb = nbytes // 34
        rows.append((first, nb, rowlen // 32, groups.index(grp), colbase, med[i]))
        first += nb
        colbase += rowlen
    return groups, rows


def sbucket(lo, hi, med):
    v = (((int(lo) | (int(hi) << 8)) - med) >> 8) + N_SB // 2
    return min(max(v, 0), N_SB - 1)


def segment_symbols(blocks, meta, colmap, b0, b1, plant=False):
    """(table, symbol) of blocks b0..b1-1 in coding order"""
    pos = np.argmax(np.abs(blocks[:, 2:].view(np.int8).astype(np.int16)), axis=1)
    firsts = [m[0] for m in meta]
    out = []
    for b in range(b0, b1):
        t = int(np.searchsorted(firsts, b, side="right")) - 1
        first, _, nb_row, grp, colbase, med = meta[t]
        inrow = (b - first) % nb_row
        base = grp * TPG
        prev = 0 if (inrow == 0 or (b == b0 and not plant)) else int(blocks[b - 1, 1])
        lo, hi, p = int(blocks[b, 0]), int(blocks[b, 1]), int(pos[b])
        out += [(base + T_HI + prev, hi), (base + T_LO + hi, lo), (base + T_POS, p), (base + T_MX, int(blocks[b, 2 + p]))]
        qb = base + T_QS + sbucket(lo, hi, med) * N_COL
        cm = colmap[colbase + inrow * 32: colbase + inrow * 32 + 32]
        out += [(qb + int(cm[j]), int(blocks[b, 2 + j])) for j in range(32) if j != p]
    return out


def normalize(counts, scale=1 << PB):
    """gpu_codec.py:193-209 as the reference writes it"""
    counts = counts.astype(np.int64)
    tot = counts.sum(1, keepdims=True)
    f = np.where(counts > 0, np.maximum(1, (counts * scale + tot // 2) // np.maximum(tot, 1)), 0)
    for r in np.nonzero(tot.ravel())[0]:
        diff = scale - f[r].sum()
        while diff != 0:
            order = np.argsort(-f[r])
            for j in order:
                if diff == 0:
                    break
                if diff > 0:
                    f[r, j] += 1; diff -= 1
                elif f[r, j] > 1:
                    f[r, j] -= 1; diff += 1
    return f.astype(np.uint16)


def rans_encode(syms, freq, cum):
    """one segment: the symbols pushed last to first; returns its bytes"""
    out = bytearray()
    x = RANS_L
    for tab, s in reversed(syms):
        f = int(freq[tab, s])
        x_max = ((RANS_L >> PB) << 8) * f
        while x >= x_max:
            out.append(x & 0xFF)
            x >>= 8
        x = ((x // f) << PB) + (x % f) + int(cum[tab, s])
    for _ in range(4):
        out.append(x & 0xFF)
        x >>= 8
    return bytes(out[::-1])


def encode(blocks, layout, plant=False):
    """-> dict(med, colmap, groups, counts, freq, lens, stream)"""
    blocks = np.asarray(blocks, np.uint8).reshape(-1, 34)
    med, colmap = stats(blocks, layout)
    groups, meta = meta_of(layout, med)
    n = len(blocks)
    segs = [segment_symbols(blocks, meta, colmap, b0, min(b0 + SEG, n), plant) for b0 in range(0, n, SEG)]
    counts = np.zeros((len(groups) * TPG, 256), np.int64)
    for syms in segs:
        if syms:
            a = np.array(syms, np.int64)
            np.add.at(counts, (a[:, 0], a[:, 1]), 1)
    freq = normalize(counts)
    cum = np.zeros((freq.shape[0], 257), np.int64)
    cum[:, 1:] = np.cumsum(freq.astype(np.int64), axis=1)
    parts = [rans_encode(s, freq, cum) for s in segs]
    return {"med": med, "colmap": colmap, "groups": groups, "counts": counts, "freq": freq,
            "lens": np.array([len(p) for p in parts], np.uint32), "stream": b"".join(parts)}
