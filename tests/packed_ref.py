"""NumPy statement of the packed low-bit format (include/crbq.h, "packed
low-bit storage"): the checker for crbq_pack / crbq_unpack.  Test
infrastructure only."""
import numpy as np

PB = 128


def key16(u):
    u = np.asarray(u, dtype=np.int64)
    return np.where(u & 0x8000, (~u) & 0xFFFF, u | 0x8000)


def unkey16(k):
    k = np.asarray(k, dtype=np.int64)
    return np.where(k & 0x8000, k & 0x7FFF, (~k) & 0xFFFF).astype(np.uint16)


NDV = 8   # distinct values a group's table is chosen from


def bits_to_f32(u, bf16):
    u = np.asarray(u, dtype=np.uint16)
    if bf16:
        return (u.astype(np.uint32) << 16).view(np.float32)
    return u.view(np.float16).astype(np.float32)


def pack_ref(qbits, masks, bf16=False, ex_cap=None):
    """qbits: uint16 [R, C] weight bit patterns; masks: uint8 [R, C] codes
    1/2/3.  Returns (codes uint8 [R, nblk*32], lut uint16 [R, nblk, 8],
    sal uint8 [nblk, 16], (ex_idx int64, ex_val uint16, ex_delta float32)
    sorted by index, status).  Per group the table keeps the `cap` most
    frequent of its NDV smallest distinct keys (ties: smaller key), in
    ascending order; other elements are exceptions coded as the group's
    first entry."""
    R, C = qbits.shape
    nblk = -(-C // PB)
    codes = np.zeros((R, nblk * 32), np.uint8)
    lut = np.zeros((R, nblk, 8), np.uint16)
    sal = np.zeros((nblk, 16), np.uint8)
    ex = []
    status = 0
    for b in range(nblk):
        c0, c1 = b * PB, min(C, b * PB + PB)
        m = masks[:, c0:c1]
        salcols = m[0] == 3
        if ((m == 3) != salcols[None, :]).any():
            status |= 2
        if ((m < 1) | (m > 3)).any():
            status |= 4
        bits = np.zeros(PB, np.uint8)
        bits[:c1 - c0] = salcols
        sal[b] = np.packbits(bits, bitorder="little")
        for r in range(R):
            k = key16(qbits[r, c0:c1])
            code = np.zeros(PB, np.int64)
            for G, cap, base in ((1, 2, 0), (2, 2, 2), (3, 4, 4)):
                sel = m[r] == G
                cand = np.unique(k[sel])[:NDV]
                cnt = np.array([(k[sel] == v).sum() for v in cand], np.int64)
                order = sorted(range(len(cand)), key=lambda i: (-cnt[i], i))[:cap]
                ks = np.sort(cand[order]) if len(order) else cand[:0]
                found = len(ks)
                for j in range(cap):
                    lut[r, b, base + j] = unkey16(ks[min(j, found - 1)]) if found else 0
                for e in np.nonzero(sel)[0]:
                    hit = np.nonzero(ks == k[e])[0]
                    rk = int(hit[0]) if len(hit) else 0
                    code[e] = (2 if G == 2 else 0) + rk
                    if not len(hit):
                        v = qbits[r, c0 + e]
                        d = bits_to_f32(v, bf16) - bits_to_f32(lut[r, b, base], bf16)
                        ex.append((r * C + c0 + e, v, np.float32(d)))
            packed = code[0::4] | (code[1::4] << 2) | (code[2::4] << 4) | (code[3::4] << 6)
            codes[r, b * 32:(b + 1) * 32] = packed.astype(np.uint8)
    cap = ex_cap if ex_cap is not None else max(1024, R * nblk // 8)
    if len(ex) > cap:
        status |= 1
    ex.sort(key=lambda t: t[0])
    exa = (np.array([t[0] for t in ex], np.int64), np.array([t[1] for t in ex], np.uint16),
           np.array([t[2] for t in ex], np.float32))
    return codes, lut, sal, exa, status


def unpack_ref(codes, lut, sal, C, ex=None):
    R = codes.shape[0]
    out = np.zeros((R, C), np.uint16)
    for c in range(C):
        b, j = divmod(c, PB)
        code = (codes[:, b * 32 + j // 4] >> (2 * (j % 4))) & 3
        s = (sal[b, j // 8] >> (j % 8)) & 1
        out[:, c] = lut[np.arange(R), b, 4 * s + code]
    if ex is not None:
        for i, v in zip(ex[0], ex[1]):
            out[i // C, i % C] = v
    return out


def structured(R, C, seed=0, dtype=np.float16, n_odd=0):
    """Weights with the binarizer's per-block structure: per block random
    salient columns shared by all rows; per row-block <= 2 values in masks
    1 and 2, <= 4 on the salient columns.  Includes a +-0 pair, groups with
    one value and an empty mask-2 group.  n_odd elements (random positions)
    then take a value outside their group's table, as an element equal to
    its group's mean does under sign(0) = 0."""
    rng = np.random.default_rng(seed)
    nblk = -(-C // PB)
    masks = np.zeros((R, C), np.uint8)
    q = np.zeros((R, C), dtype)
    for b in range(nblk):
        c0, c1 = b * PB, min(C, b * PB + PB)
        w = c1 - c0
        salcols = rng.random(w) < 0.1
        for r in range(R):
            m = np.where(salcols, 3, np.where(rng.random(w) < 0.5, 1, 2)).astype(np.uint8)
            if (r + b) % 7 == 3:
                m[m == 2] = 1                       # empty mask-2 group
            masks[r, c0:c1] = m
            vals = {G: (rng.standard_normal(4 if G == 3 else 2) * 0.05).astype(dtype)
                    for G in (1, 2, 3)}
            if (r + b) % 5 == 0:
                vals[1] = np.array([-0.0, 0.0], dtype)
            if (r + b) % 6 == 1:
                vals[2] = np.array([vals[2][0]] * 2, dtype)
            for G in (1, 2, 3):
                sel = np.nonzero(m == G)[0]
                q[r, c0 + sel] = vals[G][rng.integers(0, len(vals[G]), len(sel))]
    for _ in range(n_odd):
        r, c = int(rng.integers(0, R)), int(rng.integers(0, C))
        q[r, c] = dtype(0.0317 + 0.001 * rng.random())   # not among the planted values
    return q, masks
