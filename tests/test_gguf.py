"""CPU: the GGUF reader (miq_gguf_* in libmiq) on synthetic files.

Checks, for every file: the values and bytes the writer put there (known
answers), and -- where oracle/_ref/libsiref.so is built -- line-for-line
equality with sycl-infer's own gguf_file::load (src/model/gguf.cpp:345) over
the same file, including its error text.  The split-shard cases restate
tests/model/test_gguf_split.cpp of the reference.
"""
import os
import struct

import numpy as np
import pytest

import gguf_synth as gs

F32_T, F16_T, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 8, 12, 13, 14


# ------------------------------------------------------------------ helpers
def _val_text(v) -> str:
    if v.type == 9:
        return f"9[{len(v.arr)}](" + ";".join(_val_text(e) for e in v.arr) + ")"
    return f"{v.type}:{v.u64}:{v.i64}:{'%.17g' % v.f64}:{v.str.hex()}"


def miq_dump(miq, path) -> str:
    """The facts ref_gguf_dump prints, built from libmiq's C ABI."""
    try:
        f = miq.GgufFile(path)
    except miq.MiqError as e:
        return f"ERR {e}\n"
    with f:
        lines = [f"version {f.version}", f"split {f.split_count} {f.split_no} {len(f.shards)}"]
        lines += [f"kv {k} {_val_text(f.meta(k))}" for k in f.keys]
        for t in f.tensors:
            lines.append(f"t {t.name} {t.type} {','.join(str(d) for d in t.dims)} {t.offset} {t.map_offset} "
                         f"{t.shard}")
    return "\n".join(lines) + "\n"


def same_as_ref(miq, ref, path):
    got = miq_dump(miq, path)
    if ref is not None:
        assert got == ref.gguf_dump(str(path)), path
    return got


@pytest.fixture(scope="module")
def refopt():
    try:
        from oracle import Ref
        return Ref()
    except (FileNotFoundError, OSError):
        return None


def write(path, raw: bytes):
    with open(path, "wb") as fh:
        fh.write(raw)
    return str(path)


def all_kinds_kv():
    return [
        ("a.u8", gs.U8, 200), ("a.i8", gs.I8, -100), ("a.u16", gs.U16, 65000), ("a.i16", gs.I16, -30000),
        ("a.u32", gs.U32, 4000000000), ("a.i32", gs.I32, -2000000000), ("a.f32", gs.F32, 0.1),
        ("a.bool", gs.BOOL, 1), ("a.str", gs.STR, "héllo wörld"), ("a.u64", gs.U64, 2 ** 63 + 5),
        ("a.i64", gs.I64, -(2 ** 62)), ("a.f64", gs.F64, -1.0e300),
        ("arr.i32", gs.ARR, (gs.I32, [1, -2, 3])), ("arr.empty", gs.ARR, (gs.F32, [])),
        ("arr.str", gs.ARR, (gs.STR, ["x", "", "yz"])),
        ("arr.nested", gs.ARR, (gs.ARR, [(gs.U8, [1, 2]), (gs.STR, ["q"])])),
        ("dup", gs.U32, 1), ("dup", gs.U32, 2),
        ("general.name", gs.STR, "synthetic"), ("llama.embedding_length", gs.U32, 5120),
        ("llama.rope.freq_base", gs.F32, 1000000.0),
    ]


def some_tensors(miq, rng):
    W = (rng.standard_normal((8, 512)) * 0.02).astype(np.float32)
    return [
        ("w.q4k", (512, 8), Q4_K, miq.quantize_rows(Q4_K, W).tobytes()),
        ("w.q6k", (512, 4), Q6_K, miq.quantize_rows(Q6_K, W[:4]).tobytes()),
        ("w.q80", (512, 2, 2), Q8_0, miq.quantize_rows(Q8_0, W[:4]).tobytes()),
        ("norm", (7,), F32_T, np.arange(7, dtype=np.float32).tobytes()),
        ("emb", (3, 2, 2, 1), F16_T, np.arange(12, dtype=np.float16).tobytes()),
    ]


# ------------------------------------------------------------------ geometry
def test_type_geometry(miq, refopt):
    lib = miq.lib()
    assert (lib.miq_ggml_blck_size(Q4_K), lib.miq_ggml_type_size(Q4_K)) == (256, 144)
    assert (lib.miq_ggml_blck_size(Q8_0), lib.miq_ggml_type_size(Q8_0)) == (32, 34)
    assert lib.miq_ggml_row_bytes(Q6_K, 5120) == 20 * 210 and lib.miq_ggml_row_bytes(Q6_K, 5121) == 0
    for t in range(40):
        name = lib.miq_ggml_type_name(t).decode()
        b, z = lib.miq_ggml_blck_size(t), lib.miq_ggml_type_size(t)
        if refopt is not None:
            rn, rb, rz = refopt.ggml_geom(t)
            assert name == rn, t
            assert (b or None, z or None) == (rb, rz), t


# ------------------------------------------------------------------ single files
def test_single_file_values_and_bytes(miq, refopt, tmp_path):
    rng = np.random.default_rng(3)
    tens = some_tensors(miq, rng)
    raw, where = gs.build(all_kinds_kv(), tens, alignment=64)
    p = write(tmp_path / "m.gguf", raw)
    same_as_ref(miq, refopt, p)
    with miq.GgufFile(p) as f:
        assert f.version == 3 and not f.is_split() and f.split_count == 1 and f.split_no == 0
        assert f.map_size == len(raw) and f.data_offset % 64 == 0
        assert f.get_u32("a.u8") == 200 and f.meta("a.i8").i64 == -100
        assert f.meta("a.i8").u64 == 2 ** 64 - 100
        assert f.meta("a.u32").u64 == 4000000000 and f.meta("a.i32").i64 == -2000000000
        assert f.get_f32("a.f32") == np.float32(0.1) and f.meta("a.f64").f64 == -1.0e300
        assert f.meta("a.u64").u64 == 2 ** 63 + 5 and f.meta("a.i64").i64 == -(2 ** 62)
        assert f.get_str("a.str") == "héllo wörld" and f.get_str("nope") is None
        assert f.get_u32("nope", 77) == 77 and f.get_f32("nope", 1.5) == 1.5
        assert f.get_u32("dup") == 2  # a key written twice keeps its last value
        a = f.meta("arr.i32")
        assert a.is_arr() and a.arr_type == gs.I32 and [e.i64 for e in a.arr] == [1, -2, 3]
        assert f.meta("arr.empty").arr == [] and f.meta("arr.empty").arr_type == gs.F32
        assert [e.str for e in f.meta("arr.str").arr] == [b"x", b"", b"yz"]
        n = f.meta("arr.nested").arr
        assert [e.u64 for e in n[0].arr] == [1, 2] and n[1].arr[0].str == b"q"
        assert f.keys == sorted(f.keys)
        for name, dims, gt, data in tens:
            t = f.find(name)
            assert t is not None and t.type == gt and t.dims == dims
            assert t.nbytes == len(data) and t.map_offset == where[name]
            assert t.n_elements == int(np.prod(dims)) and t.n_rows == int(np.prod(dims[1:]))
            assert f.tensor_bytes(t).tobytes() == data
        assert f.find("missing") is None


def test_default_alignment_and_versions(miq, refopt, tmp_path):
    rng = np.random.default_rng(4)
    for ver in (1, 2, 3):
        raw, where = gs.build([("k", gs.STR, "v" * 5)], some_tensors(miq, rng)[3:], version=ver)
        p = write(tmp_path / f"v{ver}.gguf", raw)
        same_as_ref(miq, refopt, p)
        with miq.GgufFile(p) as f:
            assert f.version == ver and f.data_offset % 32 == 0
            assert all(t.map_offset == where[t.name] for t in f.tensors)


def test_header_errors(miq, refopt, tmp_path):
    rng = np.random.default_rng(5)
    raw, _ = gs.build(all_kinds_kv()[:3], some_tensors(miq, rng)[3:])
    cases = {
        "magic": b"GGUX" + raw[4:],
        # one kv pair of the unknown value type 13
        "kvtype": b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<I", 13),
        "empty": b"",
    }
    exp = {"magic": "not a gguf file", "kvtype": "gguf: unknown kv type", "empty": "mmap failed"}
    for name, b in cases.items():
        p = write(tmp_path / f"{name}.gguf", b)
        got = same_as_ref(miq, refopt, p)
        assert got == f"ERR {exp[name]}\n", (name, got)
    with pytest.raises(miq.MiqError, match="cannot open"):
        miq.GgufFile(str(tmp_path / "absent.gguf"))


def test_every_truncation_matches_reference(miq, refopt, tmp_path):
    """Every prefix of a small file: the same error (or the same parse) as the reference."""
    rng = np.random.default_rng(6)
    raw, _ = gs.build(all_kinds_kv()[8:16], some_tensors(miq, rng)[3:])
    seen = set()
    for n in range(1, len(raw) + 1):
        got = same_as_ref(miq, refopt, write(tmp_path / "cut.gguf", raw[:n]))
        seen.add(got.split("\n")[0] if got.startswith("ERR") else "ok")
    assert "ERR gguf: unexpected end of file" in seen and "ERR gguf: bad data offset" in seen and "ok" in seen


def test_random_files_match_reference(miq, refopt, tmp_path):
    if refopt is None:
        pytest.skip("oracle/_ref not built")
    rng = np.random.default_rng(7)
    scal = [gs.U8, gs.I8, gs.U16, gs.I16, gs.U32, gs.I32, gs.F32, gs.BOOL, gs.U64, gs.I64, gs.F64]
    lim = {gs.U8: (0, 255), gs.I8: (-128, 127), gs.U16: (0, 65535), gs.I16: (-32768, 32767), gs.U32: (0, 2 ** 32 - 1),
           gs.I32: (-2 ** 31, 2 ** 31 - 1), gs.BOOL: (0, 1), gs.U64: (0, 2 ** 63), gs.I64: (-2 ** 63, 2 ** 63 - 1)}

    def rand_val(t):
        if t in (gs.F32, gs.F64):
            return float(rng.standard_normal() * 10.0 ** int(rng.integers(-30, 30)))
        if t == gs.STR:
            return bytes(rng.integers(0, 256, rng.integers(0, 12), dtype=np.uint8))
        lo, hi = lim[t]
        return int(rng.integers(lo, hi, dtype=np.uint64 if lo >= 0 else np.int64, endpoint=True))

    for it in range(60):
        kv = []
        for k in range(int(rng.integers(0, 10))):
            t = int(rng.choice(scal + [gs.STR, gs.ARR]))
            if t == gs.ARR:
                et = int(rng.choice(scal + [gs.STR]))
                kv.append((f"k{k}", t, (et, [rand_val(et) for _ in range(int(rng.integers(0, 6)))])))
            else:
                kv.append((f"k{k}", t, rand_val(t)))
        tens = []
        for j in range(int(rng.integers(0, 5))):
            nd = int(rng.integers(1, 5))
            dims = tuple(int(d) for d in rng.integers(1, 5, nd))
            tens.append((f"t{j}", dims, F32_T, rng.standard_normal(int(np.prod(dims))).astype(np.float32).tobytes()))
        al = int(rng.choice([None, 8, 32, 64, 256, 4096]) or 0) or None
        raw, _ = gs.build(kv, tens, alignment=al)
        same_as_ref(miq, refopt, write(tmp_path / f"r{it}.gguf", raw))


# ------------------------------------------------------------------ split models
def test_split_metadata_only_first_shard(miq, refopt, tmp_path):
    """tests/model/test_gguf_split.cpp case 1: a 24-byte tensor-less shard 1
    whose alignment padding runs past EOF, and one F32 tensor in shard 2."""
    stem = str(tmp_path / "model")
    h0 = gs.header([], [])
    assert len(h0) == 24
    write(gs.shard_name(stem, 1, 2), h0)
    vals = np.array([1, 2, 3, 4], np.float32)
    raw, where = gs.build([], [("t", (4,), F32_T, vals.tobytes())])
    assert where["t"] == 64
    write(gs.shard_name(stem, 2, 2), raw)
    p = gs.shard_name(stem, 1, 2)
    same_as_ref(miq, refopt, p)
    with miq.GgufFile(p) as f:
        assert f.is_split() and len(f.shards) == 2 and f.split_count == 2
        t = f.find("t")
        assert t is not None and t.type == F32_T and t.n_elements == 4 and t.shard == 1
        base1, size1, _ = f.shards[1]
        assert base1 <= t.data and t.data + 16 <= base1 + size1
        assert np.array_equal(np.frombuffer(f.tensor_bytes(t), np.float32), vals)


def test_split_tensor_shard_without_data_fails(miq, refopt, tmp_path):
    """tests/model/test_gguf_split.cpp case 2: a shard that claims a tensor but ends at its header."""
    stem = str(tmp_path / "model")
    write(gs.shard_name(stem, 1, 2), gs.header([], [("t", (4,), F32_T, 0)]))
    write(gs.shard_name(stem, 2, 2), gs.header([], []))
    assert same_as_ref(miq, refopt, gs.shard_name(stem, 1, 2)) == "ERR gguf: bad data offset\n"


def split_model(miq, tmp_path, n=3, seed=8):
    rng = np.random.default_rng(seed)
    stem = str(tmp_path / "big")
    shards = []
    for i in range(n):
        kv = [("split.no", gs.U16, i), ("split.count", gs.U16, n), ("shared", gs.U32, 100 + i),
              (f"only.{i}", gs.STR, f"s{i}")]
        W = (rng.standard_normal((4 * (i + 1), 256)) * 0.02).astype(np.float32)
        tens = [(f"blk.{i}.w", (256, 4 * (i + 1)), Q4_K, miq.quantize_rows(Q4_K, W).tobytes()),
                (f"blk.{i}.b", (5 + i,), F32_T, rng.standard_normal(5 + i).astype(np.float32).tobytes())]
        raw, where = gs.build(kv, tens)
        write(gs.shard_name(stem, i + 1, n), raw)
        shards.append((raw, where, tens))
    return stem, shards


def test_split_model(miq, refopt, tmp_path):
    stem, shards = split_model(miq, tmp_path)
    for entry in (1, 2, 3):  # any shard's name opens the whole model
        p = gs.shard_name(stem, entry, 3)
        same_as_ref(miq, refopt, p)
        with miq.GgufFile(p) as f:
            assert len(f.shards) == 3 and f.split_count == 3 and f.split_no == 0
            assert f.get_u32("shared") == 100  # the first shard holding a key wins
            assert [f.get_str(f"only.{i}") for i in range(3)] == ["s0", "s1", "s2"]
            page = os.sysconf("SC_PAGESIZE")
            slot = 0
            for i, (raw, where, tens) in enumerate(shards):
                base, size, _ = f.shards[i]
                assert base - f.map_base == slot and size == len(raw)
                for name, dims, gt, data in tens:
                    t = f.find(name)
                    assert t.shard == i and t.map_offset == slot + where[name]
                    assert f.tensor_bytes(t).tobytes() == data
                slot += (len(raw) + page - 1) // page * page
            assert f.map_size == slot
            f.drop_cache(0, f.map_size)  # crosses the padding between shards


def test_split_consistency_errors(miq, refopt, tmp_path):
    stem = str(tmp_path / "bad")
    good = gs.header([("split.no", gs.U16, 1), ("split.count", gs.U16, 2)], [])
    write(gs.shard_name(stem, 1, 2), gs.header([("split.count", gs.U16, 3)], []))
    write(gs.shard_name(stem, 2, 2), good)
    assert same_as_ref(miq, refopt, gs.shard_name(stem, 1, 2)) == \
        "ERR gguf: split.count does not match the shard file names\n"
    write(gs.shard_name(stem, 1, 2), gs.header([], []))
    write(gs.shard_name(stem, 2, 2), gs.header([("split.no", gs.U16, 0)], []))
    got = same_as_ref(miq, refopt, gs.shard_name(stem, 1, 2))
    assert got.startswith("ERR gguf: shard ") and got.endswith("has split.no 0\n")
    os.remove(gs.shard_name(stem, 2, 2))
    assert same_as_ref(miq, refopt, gs.shard_name(stem, 1, 2)).startswith("ERR cannot open ")


@pytest.mark.parametrize("name", ["m-00001-of-00001.gguf", "m-0001-of-00002.gguf", "m-00001-of-0002.gguf",
                                  "m-00001-of-00002.bin", "m-0000a-of-00002.gguf", "-00001-of-00002.gguf",
                                  "m00001-of-00002.gguf", "m-00002-of-00002.gguf"])
def test_shard_name_rules(miq, refopt, tmp_path, name):
    """Which names open as one file and which as a split model (gguf.cpp:308-343)."""
    raw, _ = gs.build([("x", gs.U8, 1)], [("t", (4,), F32_T, bytes(16))])
    write(tmp_path / name, raw)
    same_as_ref(miq, refopt, str(tmp_path / name))
