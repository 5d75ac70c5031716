"""Independent packers for ggml's block formats, written from ggml's published
layouts (the block structs of ggml-common.h as documented in llama.cpp, and
the format table in gguf.mojo:15-28).  They build blocks field by field from
chosen codes and scales, so the oracle's decoders can be checked against
known answers instead of against themselves.

Q4_0  : f16 d | 16 B qs;   weight j (j<16) = low nibble of qs[j], j>=16 high nibble of qs[j-16]; w = d*(q-8)
Q4_1  : f16 d | f16 m | 16 B qs (as Q4_0);  w = d*q + m
Q8_0  : f16 d | 32 int8 qs;  w = d*q
Q4_K  : f16 d | f16 dmin | 12 B scales | 128 B qs.  Sub-block b (32 weights)
        of chunk j = b//2: weights 64j+l (l<32) are low nibbles of qs[32j+l]
        (b even), 64j+32+l high nibbles (b odd).  w = d*sc_b*q - dmin*m_b.
        6-bit scales: b<4: sc in q[b]&63, m in q[b+4]&63; b>=4: low 4 bits in
        q[b+4] (sc low nibble, m high nibble), top 2 bits in q[b-4]>>6 (sc) and
        q[b]>>6 (m).
Q5_K  : f16 d | f16 dmin | 12 B scales | 32 B qh | 128 B qs; like Q4_K plus
        bit 4 of weight 64j+l in qh[l] bit 2j, of 64j+32+l in qh[l] bit 2j+1.
Q6_K  : 128 B ql | 64 B qh | 16 int8 scales | f16 d.  Half n (128 weights):
        weight 128n+l    : ql[64n+l] low,     qh[32n+l] bits 0-1
        weight 128n+32+l : ql[64n+32+l] low,  qh[32n+l] bits 2-3
        weight 128n+64+l : ql[64n+l] high,    qh[32n+l] bits 4-5
        weight 128n+96+l : ql[64n+32+l] high, qh[32n+l] bits 6-7     (l < 32)
        w = d * sc[w // 16] * (q - 32)
"""
import numpy as np


def f16b(v):
    return np.array([v], np.float32).astype(np.float16).view(np.uint16)[0]


def f16v(v):
    return float(np.array([v], np.float32).astype(np.float16)[0])


def pack_q4_0(d, q):
    b = np.zeros(18, np.uint8)
    b[0:2] = np.array([f16b(d)], np.uint16).view(np.uint8)
    b[2:18] = (q[:16] & 0xF) | ((q[16:] & 0xF) << 4)
    return b, f16v(d) * (q.astype(np.float64) - 8)


def pack_q4_1(d, m, q):
    b = np.zeros(20, np.uint8)
    b[0:2] = np.array([f16b(d)], np.uint16).view(np.uint8)
    b[2:4] = np.array([f16b(m)], np.uint16).view(np.uint8)
    b[4:20] = (q[:16] & 0xF) | ((q[16:] & 0xF) << 4)
    return b, f16v(d) * q.astype(np.float64) + f16v(m)


def pack_q8_0(d, q):
    b = np.zeros(34, np.uint8)
    b[0:2] = np.array([f16b(d)], np.uint16).view(np.uint8)
    b[2:34] = q.astype(np.int8).view(np.uint8)
    return b, f16v(d) * q.astype(np.float64)


def pack_k_scales(sc, mn):
    """12 bytes holding 8 six-bit scales and mins."""
    q = np.zeros(12, np.uint8)
    for b in range(4):
        q[b] = (sc[b] & 63) | ((sc[b + 4] >> 4) << 6)
        q[b + 4] = (mn[b] & 63) | ((mn[b + 4] >> 4) << 6)
        q[b + 8] = (sc[b + 4] & 0xF) | ((mn[b + 4] & 0xF) << 4)
    return q


def pack_q4_k(d, dmin, sc, mn, q):
    b = np.zeros(144, np.uint8)
    b[0:2] = np.array([f16b(d)], np.uint16).view(np.uint8)
    b[2:4] = np.array([f16b(dmin)], np.uint16).view(np.uint8)
    b[4:16] = pack_k_scales(sc, mn)
    for j in range(4):
        b[16 + 32 * j:16 + 32 * j + 32] = (q[64 * j:64 * j + 32] & 0xF) | ((q[64 * j + 32:64 * j + 64] & 0xF) << 4)
    w = np.zeros(256)
    for i in range(256):
        sb = i // 32
        w[i] = f16v(d) * sc[sb] * q[i] - f16v(dmin) * mn[sb]
    return b, w


def pack_q5_k(d, dmin, sc, mn, q):
    b = np.zeros(176, np.uint8)
    b[0:2] = np.array([f16b(d)], np.uint16).view(np.uint8)
    b[2:4] = np.array([f16b(dmin)], np.uint16).view(np.uint8)
    b[4:16] = pack_k_scales(sc, mn)
    qh = np.zeros(32, np.uint8)
    for j in range(4):
        lo = q[64 * j:64 * j + 32]
        hi = q[64 * j + 32:64 * j + 64]
        b[48 + 32 * j:48 + 32 * j + 32] = (lo & 0xF) | ((hi & 0xF) << 4)
        qh |= (((lo >> 4) & 1) << (2 * j)).astype(np.uint8)
        qh |= (((hi >> 4) & 1) << (2 * j + 1)).astype(np.uint8)
    b[16:48] = qh
    w = np.zeros(256)
    for i in range(256):
        sb = i // 32
        w[i] = f16v(d) * sc[sb] * q[i] - f16v(dmin) * mn[sb]
    return b, w


def pack_q6_k(d, sc, q):
    b = np.zeros(210, np.uint8)
    for n in range(2):
        for l in range(32):
            q0, q1, q2, q3 = (int(q[128 * n + 32 * k + l]) for k in range(4))
            b[64 * n + l] = (q0 & 0xF) | ((q2 & 0xF) << 4)
            b[64 * n + 32 + l] = (q1 & 0xF) | ((q3 & 0xF) << 4)
            b[128 + 32 * n + l] = (q0 >> 4) | ((q1 >> 4) << 2) | ((q2 >> 4) << 4) | ((q3 >> 4) << 6)
    b[192:208] = np.asarray(sc, np.int8).view(np.uint8)
    b[208:210] = np.array([f16b(d)], np.uint16).view(np.uint8)
    w = np.array([f16v(d) * sc[i // 16] * (int(q[i]) - 32) for i in range(256)])
    return b, w


def random_blocks(kind, nblocks, rng):
    """Random blocks of a format as the benchmark generates them (codes
    uniform over the format's range, scales |N(0, 0.01)| as f16, 6-bit
    sub-scales uniform in [0, 63]); returns (bytes, exact float64 weights)."""
    out_b, out_w = [], []
    for _ in range(nblocks):
        d = abs(rng.normal(0, 0.01))
        if kind == "Q4_0":
            b, w = pack_q4_0(d, rng.integers(0, 16, 32))
        elif kind == "Q4_1":
            b, w = pack_q4_1(d, -abs(rng.normal(0, 0.01)), rng.integers(0, 16, 32))
        elif kind == "Q8_0":
            b, w = pack_q8_0(d, rng.integers(-128, 128, 32))
        elif kind == "Q4_K":
            b, w = pack_q4_k(d, abs(rng.normal(0, 0.01)), rng.integers(0, 64, 8), rng.integers(0, 64, 8),
                             rng.integers(0, 16, 256))
        elif kind == "Q5_K":
            b, w = pack_q5_k(d, abs(rng.normal(0, 0.01)), rng.integers(0, 64, 8), rng.integers(0, 64, 8),
                             rng.integers(0, 32, 256))
        elif kind == "Q6_K":
            b, w = pack_q6_k(d, rng.integers(-128, 128, 16), rng.integers(0, 64, 256))
        else:
            raise ValueError(kind)
        out_b.append(b)
        out_w.append(w)
    return np.concatenate(out_b), np.concatenate(out_w)
