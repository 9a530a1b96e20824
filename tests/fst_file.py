"""Writes small .fst model files for the reader tests.

The byte layout is the one scripts/fst_converter.py produces (convert_to_fst
:718-776, header :686-715 and HEADER_FMT/SHARED_ENTRY_FMT :169-172): a
128-byte little-endian header, 64-byte directory entries at the first page,
page-aligned tensor data, then the expert bank of n_layers * n_experts blocks
at a page-aligned stride; the file ends on a page boundary."""
import struct

import numpy as np

PAGE = 4096
HEADER = "<4sIIIIIIIIIIIQffQQQQQQQQ"
ENTRY = "<IHHHHIQQQQQQ"
GLOBAL = 0xFFFF
Q8_0, BF16, F32 = 1, 2, 3


def _align(x, a=PAGE):
    return (x + a - 1) // a * a


def q8_0_bytes(values):
    """Q8_0 encoding of float values: all fp16 block scales, then the int8s
    (scripts/fst_converter.py:518-536)."""
    v = np.asarray(values, np.float32).ravel()
    nb = (v.size + 31) // 32
    blocks = np.zeros(nb * 32, np.float32)
    blocks[:v.size] = v
    blocks = blocks.reshape(nb, 32)
    scale = np.abs(blocks).max(1) / 127.0
    safe = np.where(scale > 0, scale, 1.0)
    q = np.clip(np.round(blocks / safe[:, None]), -127, 127).astype(np.int8)
    return scale.astype(np.float16).tobytes() + q.tobytes()


def write_fst(path, cfg, tensors, expert_bytes, expert_block_bytes):
    """cfg: dict with hidden_dim, n_layers, n_experts, top_k, inter_dim,
    n_shared, vocab_size (and optional header fields).  tensors: list of
    (tid, lid, qtype, shape, raw bytes).  expert_bytes(l, e) -> bytes."""
    stride = _align(expert_block_bytes)
    dir_off = _align(struct.calcsize(HEADER))
    data_off = _align(dir_off + len(tensors) * struct.calcsize(ENTRY))
    entries, blobs, pos = [], [], data_off
    for tid, lid, qt, shape, raw in tensors:
        pos = _align(pos)
        s3 = (tuple(shape) + (1, 1, 1))[:3]
        entries.append(struct.pack(ENTRY, tid, lid, 0, qt, len(shape), 0, s3[0], s3[1], s3[2], pos, len(raw), 0))
        blobs.append((pos, raw))
        pos += len(raw)
    bank_off = _align(pos)
    L, E = cfg["n_layers"], cfg["n_experts"]
    with open(path, "wb") as f:
        f.write(b"\0" * data_off)
        for p, raw in blobs:
            f.seek(p)
            f.write(raw)
        for l in range(L):
            for e in range(E):
                blk = expert_bytes(l, e)
                assert len(blk) == expert_block_bytes
                f.seek(bank_off + (l * E + e) * stride)
                f.write(blk)
        f.seek(0, 2)
        f.truncate(_align(f.tell()))
        f.seek(dir_off)
        f.write(b"".join(entries))
        f.seek(0)
        f.write(struct.pack(HEADER, b"FST\0", 2, cfg["hidden_dim"], L, E, cfg["top_k"], cfg.get("n_q_heads", 32),
                            cfg.get("n_kv_heads", 4), cfg.get("head_dim", 128), cfg["inter_dim"],
                            cfg.get("n_shared", 1), 0, cfg.get("vocab_size", 0), cfg.get("rms_eps", 1e-6),
                            cfg.get("rope_freq_base", 10000.0), dir_off, len(tensors), bank_off,
                            expert_block_bytes, stride, L * E, cfg.get("dspark", 0), cfg.get("noise_id", 0)))
    return {"dir_off": dir_off, "bank_off": bank_off, "stride": stride}


def build_model(fa, path, hd=4096, inter=2048, L=2, E=8, tk=2, V=1280, seed=5, hc=True, hash_layers=0):
    """A synthetic model written as an .fst file: MXFP4 routed experts, bf16
    router [E][hd] with a bf16 bias, attention and moe norms, bf16 shared
    expert, HC control per layer and for the head, output norm and bf16 LM
    head.  Returns the arrays as written."""
    m = {"experts": {}, "router": [], "bias": [], "norm": [], "attn_norm": [], "shared": [], "hc": []}
    t = []
    for l in range(L):
        w = fa.synth_normal_bf16(seed, 100 + l, (E, hd), 0.0, 0.02)
        b = fa.synth_normal_bf16(seed, 200 + l, (E,), 0.0, 0.1)
        n = fa.synth_normal_bf16(seed, 300 + l, (hd,), 1.0, 0.1)
        an = fa.synth_normal_bf16(seed, 400 + l, (hd,), 0.5, 0.1)
        g = fa.synth_normal_bf16(seed, 500 + l, (inter, hd), 0.0, 0.02)
        u = fa.synth_normal_bf16(seed, 600 + l, (inter, hd), 0.0, 0.02)
        d = fa.synth_normal_bf16(seed, 700 + l, (hd, inter), 0.0, 0.02)
        m["router"].append(w)
        m["bias"].append(b)
        m["norm"].append(n)
        m["attn_norm"].append(an)
        m["shared"].append((g, u, d))
        t += [(3, l, BF16, (hd,), an.tobytes()), (4, l, BF16, (hd,), n.tobytes()),
              (9, l, BF16, (E, hd), w.tobytes()), (10, l, BF16, (E,), b.tobytes()),
              (11, l, BF16, (inter, hd), g.tobytes()), (12, l, BF16, (inter, hd), u.tobytes()),
              (13, l, BF16, (hd, inter), d.tobytes())]
        if hc:
            fn = fa.synth_normal_bf16(seed, 800 + l, (24, 4 * hd), 0.0, 0.02)
            sc = np.array([0.5, 0.8, 1.2], np.float32)
            bs = np.random.default_rng(seed + l).normal(0, 1, 24).astype(np.float32)
            m["hc"].append((fn, sc, bs))
            t += [(26, l, BF16, (24, 4 * hd), fn.tobytes()), (27, l, F32, (3,), sc.tobytes()),
                  (28, l, F32, (24,), bs.tobytes())]
    m["out_norm"] = fa.synth_normal_bf16(seed, 900, (hd,), 1.0, 0.1)
    m["lm_head"] = fa.synth_normal_bf16(seed, 901, (V, hd), 0.0, 0.02)
    t += [(1, GLOBAL, BF16, (hd,), m["out_norm"].tobytes()), (2, GLOBAL, BF16, (V, hd), m["lm_head"].tobytes())]
    if hc:
        hfn = fa.synth_normal_bf16(seed, 902, (4, 4 * hd), 0.0, 0.02)
        m["hc_head"] = (hfn, np.float32(0.7), np.random.default_rng(seed).normal(0, 1, 4).astype(np.float32))
        t += [(29, GLOBAL, BF16, (4, 4 * hd), hfn.tobytes()),
              (30, GLOBAL, F32, (1,), np.array([0.7], np.float32).tobytes()),
              (31, GLOBAL, F32, (4,), m["hc_head"][2].tobytes())]
    eb = 3 * hd * inter // 32 * 17

    def expert(l, e):
        blk = fa.synth_mxfp4_expert(seed, 1000 * l + e, hd, inter)
        m["experts"][(l, e)] = blk
        return blk.tobytes()

    cfg = dict(hidden_dim=hd, n_layers=L, n_experts=E, top_k=tk, inter_dim=inter, n_shared=1, vocab_size=V)
    m["layout"] = write_fst(path, cfg, t, expert, eb)
    m["tensors"] = t
    if hash_layers:
        r = np.random.default_rng(seed + 99).random((hash_layers, V, E))
        tab = np.argsort(r, axis=2)[..., :tk].astype(np.int32)  # tk distinct experts per token
        tab.tofile(str(path) + ".tid2eid")
        m["tid2eid"] = tab
    return m
