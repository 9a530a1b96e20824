"""CPU tests of the .fst reader (fst_bank_*): header fields at the offsets
ExpertPager documents (src/expert_pager.cpp:37-42, :95-100), the tensor
directory, expert addressing (ExpertPager::load_from_disk :265-290), the
context configuration, and rejection of malformed files.  No GPU needed."""
import struct

import numpy as np
import pytest

from tests import fst_file

HD, INTER, L, E, TK, V = 512, 512, 2, 3, 2, 256


@pytest.fixture(scope="module")
def model(fa, tmp_path_factory):
    path = tmp_path_factory.mktemp("fst") / "tiny.fst"
    m = fst_file.build_model(fa, path, hd=HD, inter=INTER, L=L, E=E, tk=TK, V=V, seed=3, hash_layers=2)
    m["path"] = path
    return m


def test_header_fields_and_pager_offsets(fa, model):
    raw = open(model["path"], "rb").read()
    with fa.Bank(model["path"]) as b:
        h = b.header
        assert h.magic == b"FST" and h.version == 2
        assert (h.hidden_dim, h.n_layers, h.n_experts, h.top_k, h.inter_dim) == (HD, L, E, TK, INTER)
        assert h.vocab_size == V and h.n_shared == 1
        assert abs(h.rms_eps - 1e-6) < 1e-12 and h.rope_freq_base == 10000.0
        # the fields ExpertPager reads by offset
        u32 = lambda o: struct.unpack_from("<I", raw, o)[0]
        u64 = lambda o: struct.unpack_from("<Q", raw, o)[0]
        assert (u32(4), u32(12), u32(16)) == (h.version, h.n_layers, h.n_experts)
        assert u64(80) == h.expert_bank_offset == model["layout"]["bank_off"]
        assert u64(88) == h.expert_block_bytes == 3 * HD * INTER // 32 * 17
        assert u64(96) == h.expert_block_stride == model["layout"]["stride"]
        assert h.expert_block_stride % 4096 == 0 and h.expert_block_stride >= h.expert_block_bytes
        assert u64(104) == h.expert_count == L * E
        assert h.shared_dir_count == len(model["tensors"])
        assert len(raw) % 4096 == 0


def test_directory_and_tensor_bytes(fa, model):
    with fa.Bank(model["path"]) as b:
        ts = b.tensors()
        assert len(ts) == len(model["tensors"])
        for t, (tid, lid, qt, shape, data) in zip(ts, model["tensors"]):
            s3 = (tuple(shape) + (1, 1, 1))[:3]
            assert (t.tid, t.lid, t.qtype, t.ndim, tuple(t.shape)) == (tid, lid, qt, len(shape), s3)
            assert t.offset % 4096 == 0 and t.size == len(data)
            assert b.read_tensor(t).tobytes() == data
        # by (tid, layer): the layer's own entry, not another layer's
        r1 = b.find(9, 1)
        assert b.read_tensor(r1).tobytes() == model["router"][1].tobytes()
        assert b.read_tensor(b.find(4, 0)).tobytes() == model["norm"][0].tobytes()
        assert b.read_tensor(b.find(3, 0)).tobytes() == model["attn_norm"][0].tobytes()
        assert b.read_tensor(b.find(2)).tobytes() == model["lm_head"].tobytes()
        with pytest.raises(fa.FstError) as e:
            b.find(9, 5)
        assert e.value.code == fa.FST_ENOTREADY


def test_expert_addressing(fa, model):
    with fa.Bank(model["path"]) as b:
        raw = open(model["path"], "rb").read()
        h = b.header
        for l in range(L):
            for e in range(E):
                blk = b.read_expert(l, e)
                assert np.array_equal(blk, model["experts"][(l, e)])
                off = h.expert_bank_offset + (l * E + e) * h.expert_block_stride
                assert raw[off:off + h.expert_block_bytes] == blk.tobytes()
        for bad in ((L, 0), (0, E), (-1, 0)):
            with pytest.raises(fa.FstError):
                b.read_expert(*bad)


def test_bank_config(fa, model):
    with fa.Bank(model["path"]) as b:
        c = b.config(max_tokens=32)
        assert (c.hidden_dim, c.inter_dim, c.n_experts, c.top_k, c.n_layers, c.vocab_size) == (HD, INTER, E, TK, L, V)
        assert c.codec == fa.CODEC_MXFP4 and c.has_shared == 1 and c.max_tokens == 32
        assert c.score_func == fa.SCORE_SQRTSOFTPLUS and abs(c.route_scale - 1.5) < 1e-7
        assert c.n_hash_layers == 3 and c.round_logits_bf16 == 1 and c.swiglu_limit == 0.0
        assert fa.expert_bytes(c) == b.header.expert_block_bytes


def _patched(src, dst, off, fmt, value):
    raw = bytearray(open(src, "rb").read())
    struct.pack_into(fmt, raw, off, value)
    open(dst, "wb").write(raw)


def test_malformed_files_rejected(fa, model, tmp_path):
    src = model["path"]
    raw = open(src, "rb").read()
    cases = {
        "magic": lambda p: open(p, "wb").write(b"GGUF" + raw[4:]),
        "short": lambda p: open(p, "wb").write(raw[:100]),
        "truncated_bank": lambda p: open(p, "wb").write(raw[:len(raw) - 4096 * 40]),
        "dir_past_eof": lambda p: _patched(src, p, 64, "<Q", len(raw)),
        "tensor_past_eof": lambda p: _patched(src, p, 4096 + 40, "<Q", len(raw) - 16),
        "stride_lt_block": lambda p: _patched(src, p, 96, "<Q", 1024),
    }
    for name, make in cases.items():
        p = tmp_path / (name + ".fst")
        make(p)
        with pytest.raises(fa.FstError):
            fa.Bank(p)
    with pytest.raises(fa.FstError):
        fa.Bank(tmp_path / "missing.fst")
    # a block size that is not an MXFP4 expert of the geometry
    p = tmp_path / "eb.fst"
    _patched(src, p, 88, "<Q", 3 * HD * INTER // 32 * 17 - 4096)
    with fa.Bank(p) as b:
        with pytest.raises(fa.FstError):
            b.config()
