"""The .qnt loader (quanta.cpp_amd/qnt.py: read_qnt, check_model, load_model) on good and malformed files.

Every malformed file is refused with the message the reference's own loader gives for it (ModelFile::open,
engine/src/model_file.cpp:104-218; Model::load, engine/src/model.cpp:10-58): where the reference build is present
(oracle/_ref), each case is also loaded by the reference's Model::load and the two messages must be equal."""
import struct

import numpy as np
import pytest

from decoder_util import qnt_module

qnt = qnt_module()
HP = qnt.HParams(vocab_size=512, dim=128, n_layers=2, n_heads=2, n_kv_heads=1, head_dim=64, ffn_dim=256, max_seq=64)


@pytest.fixture(scope="module")
def model():
    return qnt.synthetic_q4mix(3, HP)


@pytest.fixture(scope="module")
def good_file(model, tmp_path_factory):
    path = str(tmp_path_factory.mktemp("qnt") / "good.qnt")
    qnt.write_qnt(path, HP, model)
    return path


def reference_verdict(path):
    import oracle as o
    if o.ref is None:
        return "unchecked"
    return o.ref.load_error(path)


def refused(path, message):
    with pytest.raises(qnt.QntError) as e:
        qnt.load_model(path)
    assert str(e.value) == message
    ref = reference_verdict(path)
    assert ref in ("unchecked", message), f"the reference says {ref!r}"


def table_entry_offset(data: bytes, name: str) -> int:
    """Byte offset of a tensor's table entry (its name's length prefix) in a file's bytes."""
    key = struct.pack("<I", len(name)) + name.encode()
    i = data.find(key)
    assert i > 0
    return i


def test_round_trip(model, good_file):
    hp, n_tokens, tens = qnt.load_model(good_file)
    assert n_tokens == HP.vocab_size and (hp.vocab_size, hp.dim, hp.n_layers, hp.ffn_dim) == (512, 128, 2, 256)
    assert set(tens) == set(model)
    for name, rec in model.items():
        got = tens[name]
        assert (got.dtype, got.rows, got.cols, got.ndim) == (rec.dtype, rec.rows, rec.cols, rec.ndim), name
        assert np.array_equal(np.asarray(got.data), rec.data), name
    assert reference_verdict(good_file) in ("unchecked", None)


def test_bad_magic_and_version(good_file, tmp_path):
    data = bytearray(open(good_file, "rb").read())
    p = tmp_path / "m.qnt"
    p.write_bytes(b"QNT2" + data[4:])
    refused(str(p), "bad magic (not a .qnt file)")
    for v in (0, 3):
        p.write_bytes(data[:4] + struct.pack("<I", v) + data[8:])
        refused(str(p), f"unsupported version {v}")
    p.write_bytes(data[:3])
    refused(str(p), "model file truncated")


@pytest.mark.parametrize("cut", [6, 30, 60, 200])
def test_truncated_header_and_tokenizer(good_file, tmp_path, cut):
    data = open(good_file, "rb").read()
    p = tmp_path / "m.qnt"
    p.write_bytes(data[:cut])
    refused(str(p), "model file truncated")


def test_tokenizer_section_shorter_than_its_tokens(good_file, tmp_path):
    """The tokenizer section's own length says less than its token strings need: its cursor runs out."""
    data = bytearray(open(good_file, "rb").read())
    at = 4 + 4 + 52  # magic, version, hparams (version 2)
    n = struct.unpack_from("<I", data, at)[0]
    struct.pack_into("<I", data, at, n - 100)
    p = tmp_path / "m.qnt"
    p.write_bytes(bytes(data))
    refused(str(p), "model file truncated")


def test_truncated_tensor_data(good_file, tmp_path):
    data = open(good_file, "rb").read()
    hp, _, tens = qnt.read_qnt(good_file)
    # the tensor whose data ends last
    last = max(tens, key=lambda n: tens[n].data.ctypes.data + tens[n].data.size)
    p = tmp_path / "m.qnt"
    p.write_bytes(data[:-10])
    refused(str(p), f"tensor out of bounds: {last}")


def test_bad_offset_and_ndim(good_file, tmp_path):
    data = bytearray(open(good_file, "rb").read())
    name = "model.layers.1.mlp.up_proj.weight"
    at = table_entry_offset(bytes(data), name) + 4 + len(name)
    dtype, ndim = struct.unpack_from("<II", data, at)
    assert ndim == 2
    off_at = at + 8 + 8
    bad = bytearray(data)
    struct.pack_into("<Q", bad, off_at, len(data) + 64)
    p = tmp_path / "m.qnt"
    p.write_bytes(bytes(bad))
    refused(str(p), f"bad offset for {name}")
    bad = bytearray(data)
    struct.pack_into("<Q", bad, off_at, len(data) - 100)
    p.write_bytes(bytes(bad))
    refused(str(p), f"tensor out of bounds: {name}")
    bad = bytearray(data)
    struct.pack_into("<I", bad, at + 4, 3)
    p.write_bytes(bytes(bad))
    refused(str(p), f"unsupported ndim for {name}")


def test_missing_tensor(model, tmp_path):
    for name in ("model.layers.1.mlp.up_proj.weight", "model.norm.weight", "model.layers.0.self_attn.k_proj.bias"):
        t = {k: v for k, v in model.items() if k != name}
        p = str(tmp_path / "m.qnt")
        qnt.write_qnt(p, HP, t)
        refused(p, f"missing tensor: {name}")


def test_bad_shortlist_tensors(model, tmp_path):
    p = str(tmp_path / "m.qnt")
    t = {k: v for k, v in model.items() if k != "quanta.head_err"}
    qnt.write_qnt(p, HP, t)
    refused(p, "bad shortlist head tensors")
    t = dict(model)
    e = model["quanta.head_err"]
    t["quanta.head_err"] = qnt.TensorRec(e.dtype, e.rows // 2, e.cols, e.data[: e.data.size // 2])
    qnt.write_qnt(p, HP, t)
    refused(p, "bad shortlist head tensors")
    t = dict(model)
    h = model["quanta.head_q4"]
    t["quanta.head_q4"] = qnt.TensorRec(qnt.Q8_0, h.rows, h.cols // 2, h.data)
    qnt.write_qnt(p, HP, t)
    refused(p, "bad shortlist head tensors")


def test_bad_head_configuration(model, tmp_path):
    p = str(tmp_path / "m.qnt")
    bad = qnt.HParams(**{**HP.__dict__, "n_heads": 3})
    qnt.write_qnt(p, bad, model)
    refused(p, "unsupported head configuration")


def test_untied_head_and_hadamard_load(model, tmp_path):
    """An untied LM head (lm_head.weight) and the Hadamard-rotated down projection load as the reference loads them;
    the Hadamard flag still needs ffn_dim % 256 == 0 (model.cpp:39-42), and an untied file needs its lm_head.weight."""
    p = str(tmp_path / "m.qnt")
    t = dict(model)
    t["lm_head.weight"] = model["model.embed_tokens.weight"]
    untied = qnt.HParams(**{**HP.__dict__, "tied_embeddings": False})
    qnt.write_qnt(p, untied, t)
    assert reference_verdict(p) in ("ok", "unchecked", None)
    hp, _, tens = qnt.load_model(p)
    assert not hp.tied_embeddings and "lm_head.weight" in tens
    qnt.write_qnt(p, untied, model)
    refused(p, "missing tensor: lm_head.weight")
    qnt.write_qnt(p, qnt.HParams(**{**HP.__dict__, "flags": qnt.FLAG_HADAMARD_DOWN}), model)
    assert reference_verdict(p) in ("ok", "unchecked", None)
    hp, _, _ = qnt.load_model(p)
    assert hp.flags == qnt.FLAG_HADAMARD_DOWN
    qnt.write_qnt(p, qnt.HParams(**{**HP.__dict__, "flags": qnt.FLAG_HADAMARD_DOWN, "ffn_dim": 160}), model)
    refused(p, "hadamard flag needs ffn_dim % 256 == 0")
