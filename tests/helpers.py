"""Shared test helpers (closed-form encoders, error metrics)."""
import numpy as np


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def bf16_to_f32(a):
    return (np.asarray(a, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(a):
    u = np.asarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def pack_scale_min(sc, m):
    """Inverse of get_scale_min_k4 (ggml Q4_K packing of eight 6-bit scales and
    mins into 12 bytes): j<4 live in the low 6 bits of bytes j (sc) and j+4 (m);
    j>=4 keep their low 4 bits in byte j+4 (sc low nibble, m high nibble) and
    their top 2 bits in the top bits of bytes j-4 (sc) and j (m)."""
    q = [0] * 12
    for j in range(8):
        s, mm = int(sc[j]), int(m[j])
        assert 0 <= s < 64 and 0 <= mm < 64
        if j < 4:
            q[j] |= s
            q[j + 4] |= mm
        else:
            q[j + 4] |= (s & 15) | ((mm & 15) << 4)
            q[j - 4] |= (s >> 4) << 6
            q[j] |= (mm >> 4) << 6
    return np.array(q, np.uint8)


def make_q4k_block(d16, dmin16, sc, m, q):
    """q: 256 nibble values in element order.  Element 64g+i is the low nibble
    of qs[32g+i], element 64g+32+i its high nibble."""
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.frombuffer(np.uint16(d16).tobytes(), np.uint8)
    blk[2:4] = np.frombuffer(np.uint16(dmin16).tobytes(), np.uint8)
    blk[4:16] = pack_scale_min(sc, m)
    q = np.asarray(q, np.uint8)
    for g in range(4):
        lo = q[64 * g: 64 * g + 32]
        hi = q[64 * g + 32: 64 * g + 64]
        blk[16 + 32 * g: 16 + 32 * g + 32] = lo | (hi << 4)
    return blk


def q4k_closed_form(d, dmin, sc, m, q):
    """w = d*sc_j*q - dmin*m_j for element i in sub-block j = i // 32 (float64)."""
    j = np.arange(256) // 32
    return d * np.asarray(sc, np.float64)[j] * np.asarray(q, np.float64) - dmin * np.asarray(m, np.float64)[j]
