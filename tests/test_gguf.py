"""The GGUF tensor locator (bpd_substrate_amd/gguf.py): the reference's
malformed-file fixtures (tests/crossword_attacks/, copied to
tests/golden/gguf/), round trips through the writer, and robustness of the
walk against truncated and corrupted bytes.  CPU only."""
import os
import random
import struct

import numpy as np
import pytest

from bpd_substrate_amd import gguf, synth

HERE = os.path.dirname(os.path.abspath(__file__))
FIX = os.path.join(HERE, "golden", "gguf")

# fixture -> failing checks of gguf.report (the reference's own checks,
# lib/gguf_validate.pl:74-95, plus this locator's structural ones)
EXPECTED = {
    "valid_model.gguf": set(),
    "missing_rope_params.gguf": {"rope_params"},
    # Q4_0 weight and Q4_K bias in one layer; K-quant without a version; llama without
    # rope keys; and a 64-element Q4_K row, which is not a whole number of blocks
    "mixed_quant_layer.gguf": {"type_consistency", "quant_version", "rope_params", "block_shape"},
    "wrong_quant_version.gguf": {"quant_version", "rope_params", "block_shape"},
    # the walk itself fails on these
    "key_length_overflow.gguf": {"parse"},
    "string_length_overflow.gguf": {"parse"},
    "string_into_tensor_data.gguf": {"parse"},
    "tensor_header_overlap.gguf": {"parse"},
    "tensor_tensor_overlap.gguf": {"parse"},
}


@pytest.mark.parametrize("name", sorted(EXPECTED))
def test_reference_fixtures(name):
    rep = gguf.report(os.path.join(FIX, name))
    failing = {c for c, ok, _ in rep if not ok}
    assert failing == EXPECTED[name], rep


def test_fixture_failure_reasons():
    why = lambda n: dict((c, d) for c, ok, d in gguf.report(os.path.join(FIX, n)) if not ok)["parse"]
    assert "shares bytes" in why("tensor_tensor_overlap.gguf")
    assert "past the end" in why("tensor_header_overlap.gguf")
    assert "key 0" in why("key_length_overflow.gguf")
    assert "general.architecture" in why("string_length_overflow.gguf")


def test_valid_fixture_layout():
    g = gguf.open_gguf(os.path.join(FIX, "valid_model.gguf"))
    assert g.version == 3 and g.alignment == 32
    (t,) = g.tensors
    assert (t.name, t.dims, t.type_name) == ("token_embd.weight", (64, 256), "F32")
    assert t.abs_offset == g.data_start and g.data_start % 32 == 0
    assert t.abs_offset + t.nbytes == g.file_size and g.unclaimed == []


def test_strict_open_rejects_what_report_flags():
    for name in ("mixed_quant_layer.gguf", "wrong_quant_version.gguf"):
        with pytest.raises(gguf.GGUFError, match="not a multiple"):
            gguf.open_gguf(os.path.join(FIX, name))
    with pytest.raises(gguf.GGUFError, match="alignment"):
        gguf.open_gguf(os.path.join(FIX, "tensor_tensor_overlap.gguf"))


def _model(path, alignment=32):
    w = synth.q4k(16, 512, synth.key(60, 1))
    q = synth.q8_0(8, 128, synth.key(60, 2))
    f = synth.normal_f32(64, synth.key(60, 3))
    meta = [("general.architecture", gguf.T_STR, "llama"), ("llama.rope.freq_base", gguf.T_F32, 10000.0),
            ("general.quantization_version", gguf.T_U32, 3), ("llama.block_count", gguf.T_U32, 1),
            ("tokenizer.ggml.tokens", gguf.T_ARR, (gguf.T_STR, ["<s>", "a", "", "zz"])),
            ("tokenizer.ggml.scores", gguf.T_ARR, (gguf.T_F32, [0.0, -1.5, 2.0, 3.25])),
            ("general.flag", gguf.T_BOOL, True), ("general.big", gguf.T_U64, 2 ** 40)]
    tensors = [("blk.0.ffn_gate.weight", (512, 16), gguf.Q4_K, w.tobytes()),
               ("token_embd.weight", (128, 8), gguf.Q8_0, q.tobytes()),
               ("output_norm.weight", (64,), 0, f.tobytes())]
    gguf.write_gguf(path, meta, tensors, alignment=alignment)
    return tensors


@pytest.mark.parametrize("alignment", [32, 64, 256])
def test_round_trip(tmp_path, alignment):
    p = str(tmp_path / "m.gguf")
    tensors = _model(p, alignment)
    g = gguf.open_gguf(p)
    assert g.alignment == alignment
    assert g.metadata["tokenizer.ggml.tokens"] == ["<s>", "a", "", "zz"]
    assert g.metadata["tokenizer.ggml.scores"] == [0.0, -1.5, 2.0, 3.25]
    assert g.metadata["general.big"] == 2 ** 40 and g.metadata["general.flag"] is True
    for name, dims, ttype, data in tensors:
        t = g.tensor(name)
        assert t.dims == dims and t.type == ttype and t.abs_offset % alignment == 0
        assert bytes(g.tensor_bytes(name)) == data
    assert g.tensor("blk.0.ffn_gate.weight").nbytes == 16 * 2 * 144
    assert g.tensor("token_embd.weight").nbytes == 8 * 4 * 34
    assert all(ok for _, ok, _ in gguf.report(p))


def test_exact_sizes_of_the_path_types():
    assert gguf.tensor_nbytes((4096, 14336), gguf.Q4_K) == 33030144   # the headline metric shape
    assert gguf.tensor_nbytes((4096, 14336), gguf.Q8_0) == 62390272   # cfg2
    assert gguf.tensor_nbytes((4096, 4096), gguf.Q6_K) == 4096 * 16 * 210
    with pytest.raises(gguf.GGUFError):
        gguf.tensor_nbytes((100,), gguf.Q8_0)
    with pytest.raises(gguf.GGUFError):
        gguf.tensor_nbytes((32,), 99)


def test_every_truncation_is_rejected_cleanly(tmp_path):
    p = str(tmp_path / "m.gguf")
    _model(p)
    full = open(p, "rb").read()
    g = gguf.parse(full)
    end = max(t.abs_offset + t.nbytes for t in g.tensors)
    for n in range(0, end):
        with pytest.raises(gguf.GGUFError):
            gguf.parse(full[:n])


def test_corrupted_bytes_never_escape_as_other_errors(tmp_path):
    """Random byte flips in the header region: the walk either parses or raises
    GGUFError, never another exception, and never claims a byte twice."""
    p = str(tmp_path / "m.gguf")
    _model(p)
    full = bytearray(open(p, "rb").read())
    head = gguf.parse(bytes(full)).data_start
    rng = random.Random(7)
    for _ in range(3000):
        b = bytearray(full)
        for _ in range(rng.randint(1, 4)):
            b[rng.randrange(head)] = rng.randrange(256)
        try:
            g = gguf.parse(bytes(b), strict=False)
        except gguf.GGUFError:
            continue
        spans = sorted((t.abs_offset, t.abs_offset + t.nbytes) for t in g.tensors)
        assert all(e <= s for (_, e), (s, _) in zip(spans, spans[1:]))
        assert all(e <= len(b) for _, e in spans)


def test_huge_counts_are_bounded_before_allocation():
    hdr = struct.pack("<IIQQ", gguf.MAGIC, 3, 2 ** 40, 2 ** 40)
    with pytest.raises(gguf.GGUFError, match="cannot fit"):
        gguf.parse(hdr + b"\0" * 64)
    # an array whose count cannot fit in the file
    kv = struct.pack("<Q", 1) + b"k" + struct.pack("<IIQ", gguf.T_ARR, gguf.T_U32, 2 ** 50)
    with pytest.raises(gguf.GGUFError, match="cannot fit"):
        gguf.parse(struct.pack("<IIQQ", gguf.MAGIC, 3, 0, 1) + kv + b"\0" * 64)


def test_bad_magic_version_alignment_and_duplicates(tmp_path):
    with pytest.raises(gguf.GGUFError, match="magic"):
        gguf.parse(b"GGUX" + b"\0" * 60)
    with pytest.raises(gguf.GGUFError, match="version"):
        gguf.parse(struct.pack("<IIQQ", gguf.MAGIC, 1, 0, 0))
    p = str(tmp_path / "a.gguf")
    gguf.write_gguf(p, [("general.alignment", gguf.T_U32, 48)], [])
    with pytest.raises(gguf.GGUFError, match="power of two"):
        gguf.open_gguf(p)
    one = np.zeros(4, np.float32).tobytes()
    gguf.write_gguf(p, [], [("t", (4,), 0, one), ("t", (4,), 0, one)])
    with pytest.raises(gguf.GGUFError, match="duplicate tensor"):
        gguf.open_gguf(p)


def _qv_file(path, ttype, nbytes, qv):
    meta = [("general.architecture", gguf.T_STR, "llama"), ("llama.rope.freq_base", gguf.T_F32, 10000.0)]
    if qv is not None:
        meta.append(("general.quantization_version",) + qv)
    gguf.write_gguf(path, meta, [("blk.0.ffn_up.weight", (256, 1), ttype, bytes(nbytes))])
    return dict((c, (ok, d)) for c, ok, d in gguf.report(path))


def test_quant_version_covers_exactly_the_reference_kquant_types(tmp_path):
    # lib/gguf_validate.pl:148-152: kquant_type is 12..15.  Q2_K / Q3_K files do not need
    # quantization_version >= 3; a Q4_K file does.
    p = str(tmp_path / "q.gguf")
    assert _qv_file(p, 11, 110, (gguf.T_U32, 2))["quant_version"][0]           # Q3_K, version 2
    assert _qv_file(p, 10, 84, None)["quant_version"][0]                      # Q2_K, no version
    assert not _qv_file(p, 12, 144, (gguf.T_U32, 2))["quant_version"][0]      # Q4_K, version 2
    assert _qv_file(p, 15, 292, (gguf.T_U32, 3))["quant_version"][0]          # Q8_K, version 3


def test_non_numeric_quant_version_is_a_failed_check(tmp_path):
    p = str(tmp_path / "q.gguf")
    ok, detail = _qv_file(p, 12, 144, (gguf.T_STR, "3"))["quant_version"]
    assert not ok and "not a number" in detail
