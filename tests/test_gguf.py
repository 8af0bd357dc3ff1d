"""The GGUF reader (q35m_gguf_*) on files written to the published layout by
tests/gguf_writer.py: metadata of every scalar type, arrays skipped, tensor
infos and data at the default (32) and a custom alignment, and the errors
GgufFile raises (GgufFile.cs:110-170: magic, version 2-3, non-power-of-two
alignment, a data section past the end).  Runs without a device."""
import numpy as np
import pytest

import gguf_writer as gw
import q35mix


def test_metadata_and_tensors(tmp_path):
    p = tmp_path / "a.gguf"
    w = np.arange(24, dtype=np.float32).reshape(4, 6)
    q = np.arange(144 * 2, dtype=np.uint8)
    kv = [("general.architecture", gw.STRING, "qwen35"), ("qwen35.block_count", gw.U32, 2),
          ("x.i8", gw.I8, -5), ("x.u64", gw.U64, 1 << 40), ("x.f32", gw.F32, 0.5), ("x.f64", gw.F64, -2.25),
          ("x.bool", gw.BOOL, 1), ("x.arr", gw.ARRAY, (gw.I32, [1, 2, 3])),
          ("x.strs", gw.ARRAY, (gw.STRING, ["a", "bc"]))]
    for align in (None, 64):
        gw.write(p, kv, [gw.f32("blk.0.ssm_a", w), ("blk.0.q", 12, (512,), q.tobytes())], alignment=align)
        g = q35mix.Gguf(p)
        assert g.string("general.architecture") == "qwen35"
        assert g.int("qwen35.block_count") == 2 and g.int("x.i8") == -5 and g.int("x.u64") == 1 << 40
        assert g.int("x.bool") == 1
        assert g.float("x.f32") == 0.5 and g.float("x.f64") == -2.25
        t, dims, raw = g.tensor("blk.0.ssm_a")
        assert t == 0 and dims == (6, 4) and np.array_equal(np.frombuffer(raw, np.float32).reshape(4, 6), w)
        t, dims, raw = g.tensor("blk.0.q")
        assert t == 12 and dims == (512,) and raw == q.tobytes()
        with pytest.raises(q35mix.Q35Error) as e:
            g.tensor("nope")
        assert e.value.code == q35mix.ERR_RANGE
        with pytest.raises(q35mix.Q35Error):
            g.int("x.f32")
        g.close()


@pytest.mark.parametrize("case,code", [("magic", "INVALID"), ("version", "UNSUPPORTED"),
                                       ("align", "INVALID"), ("short", "INVALID"), ("falign", "INVALID")])
def test_rejects_bad_files(tmp_path, case, code):
    p = tmp_path / "b.gguf"
    t = [gw.f32("t", np.ones(8, np.float32))]
    if case == "magic":
        gw.write(p, [], t, magic=b"GGUX")
    elif case == "version":
        gw.write(p, [], t, version=4)
    elif case == "align":
        gw.write(p, [], t, alignment=48)
    elif case == "falign":
        gw.write(p, [("general.alignment", gw.F64, 32.0)], t)
    else:
        gw.write(p, [("k", gw.STRING, "v" * 100)], t)
        p.write_bytes(p.read_bytes()[:60])
    with pytest.raises(q35mix.Q35Error) as e:
        q35mix.Gguf(p)
    assert e.value.code == getattr(q35mix, "ERR_" + code)


def test_tensor_extent_checks(tmp_path):
    """q35m_gguf_tensor refuses a tensor whose element count overflows 64 bits
    and a tensor (of a type the reader sizes or not) whose offset lies past
    the end of the file, rather than returning a pointer outside the mapping."""
    p = tmp_path / "c.gguf"
    ok = gw.f32("ok", np.ones(8, np.float32))
    huge = ("huge", 0, (1 << 40, 1 << 40), b"")            # 2^80 F32 elements
    far_f32 = ("far_f32", 0, (8,), b"")                     # F32 at a far offset
    far_q40 = ("far_q40", 2, (32,), b"")                    # Q4_0: not sized by the reader
    gw.write(p, [], [ok, huge, far_f32, far_q40], offsets=[0, 0, 1 << 30, 1 << 30])
    g = q35mix.Gguf(p)
    t, dims, raw = g.tensor("ok")
    assert t == 0 and np.array_equal(np.frombuffer(raw, np.float32), np.ones(8, np.float32))
    for name in ("huge", "far_f32", "far_q40"):
        with pytest.raises(q35mix.Q35Error) as e:
            g.tensor(name)
        assert e.value.code == q35mix.ERR_INVALID, name
    g.close()


def test_legacy_stride16_type42_is_stq1_0(tmp_path):
    """GgufTypeTests.LegacyStride16Type42IsNormalizedWithoutBreakingQ2
    (tests/Qwen35Sharp.Tests/GgufTypeTests.cs:8-29): raw type 42 in a file
    with general.file_type 41 named "... Stride16" reads as STQ1_0 (43, sized
    at 42 bytes a 256-value block); in a plain file it stays 42 (Q2_0)."""
    for name, want in (("Hy-MT2 1.25Bit Stride16", 43), ("plain Q2 model", 42), ("x stride16 y", 43)):
        p = tmp_path / "t.gguf"
        gw.write(p, [("general.name", gw.STRING, name), ("general.file_type", gw.I32, 41)],
                 [("x", 42, (256,), bytes(range(64)))])
        g = q35mix.Gguf(p)
        t, dims, raw = g.tensor("x")
        assert t == want and dims == (256,), name
        if want == 43:
            assert raw == bytes(range(42))
        g.close()
    gw.write(p, [("general.name", gw.STRING, "Stride16"), ("general.file_type", gw.I32, 40)],
             [("x", 42, (256,), bytes(64))])
    g = q35mix.Gguf(p)
    assert g.tensor("x")[0] == 42
    g.close()
