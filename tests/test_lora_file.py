"""The 'LORA' v1 adapter binary (include/glacier_lora_file.h): the byte layout
of GgufLoraModel.SaveAdapter / TuneBlockSerialization.WriteTensor
(GgufLoraModel.cs:636-650, ITuneBlock.cs:43-50), built here independently with
struct and the .NET BinaryWriter 7-bit string length, and the reader's checks
of GgufLoraModel.LoadAdapter (:697-796).  Host code only."""
import os
import struct

import numpy as np
import pytest

import glacier_attn as ga


def _dotnet_string(s):
    """BinaryWriter.Write(string): UTF-8 byte count as a 7-bit varint, then the bytes."""
    b = s.encode("utf-8")
    n, out = len(b), bytearray()
    while n >= 0x80:
        out.append((n | 0x80) & 0xFF)
        n >>= 7
    out.append(n)
    return bytes(out) + b


def _record(name, a):
    a = np.ascontiguousarray(a, np.float32)
    return _dotnet_string(name) + struct.pack("<ii", *a.shape) + a.tobytes()


def _file(layer_count, rank, alpha, records, count=None, magic=0x41524F4C, version=1):
    head = struct.pack("<IIiifi", magic, version, layer_count, rank, alpha,
                       len(records) if count is None else count)
    return head + b"".join(records)


def _tensors(seed=0, rank=4, d_in=16, d_out=24):
    rng = np.random.default_rng(seed)
    out = []
    for proj in ("attn_q", "attn_v"):
        out.append((f"blk.0.{proj}.lora_a.weight", rng.standard_normal((d_in, rank)).astype(np.float32)))
        out.append((f"blk.0.{proj}.lora_b.weight", rng.standard_normal((rank, d_out)).astype(np.float32)))
    return out


def test_saved_bytes_match_the_reference_layout(tmp_path):
    ts = _tensors()
    path = tmp_path / "adapter_model.bin"
    ga.lora_save(path, 1, 4, 8.0, ts)
    want = _file(1, 4, 8.0, [_record(n, a) for n, a in ts])
    assert path.read_bytes() == want
    assert not os.path.exists(str(path) + ".tmp")


def test_round_trip_and_directory_path(tmp_path):
    ts = _tensors(seed=1)
    ga.lora_save(tmp_path / "adapter_model.bin", 2, 4, 16.0, ts)
    for p in (tmp_path / "adapter_model.bin", tmp_path):  # a directory means <dir>/adapter_model.bin
        hdr, got = ga.lora_load(p)
        assert hdr == {"version": 1, "layer_count": 2, "rank": 4, "alpha": 16.0, "tensor_count": 4}
        assert [n for n, _ in got] == [n for n, _ in ts]
        for (_, a), (_, b) in zip(ts, got):
            assert np.array_equal(a, b)


def test_transposed_layout_reads_back_native(tmp_path):
    """As the reference test's WriteTransposedAdapterBinary
    (GradientAndGpuParityTests.cs:690-716): records stored [dim1][dim0]."""
    ts = _tensors(seed=2)
    raw = _file(1, 4, 8.0, [_record(n, a.T) for n, a in ts])
    p = tmp_path / "t.bin"
    p.write_bytes(raw)
    _, got = ga.lora_load(p, transpose=lambda name, d0, d1: True)
    for (_, a), (_, b) in zip(ts, got):
        assert np.array_equal(a, b)


def test_long_names_use_a_two_byte_length(tmp_path):
    name = "blk.0." + "x" * 200 + ".lora_a.weight"
    a = np.arange(6, dtype=np.float32).reshape(2, 3)
    ga.lora_save(tmp_path / "a.bin", 1, 2, 4.0, [(name, a)])
    raw = (tmp_path / "a.bin").read_bytes()
    assert raw[24:26] == bytes([(len(name) | 0x80) & 0xFF, len(name) >> 7])
    _, got = ga.lora_load(tmp_path / "a.bin")
    assert got[0][0] == name and np.array_equal(got[0][1], a)


def test_the_reference_corrupted_dims_fixture_reads_as_written(tmp_path):
    """GgufMerger_SafetyGuards_RejectInPlaceOverwriteAndCorruptedAdapterDimensions
    (GradientAndGpuParityTests.cs:556-576) writes a well-formed file whose A
    has the wrong in-dimension for the model: the file reader returns it as
    written, and matching it to a model is the caller's check."""
    raw = _file(1, 4, 8.0, [_record("blk.0.attn_q.lora_a.weight", np.zeros((32, 4))),
                            _record("blk.0.attn_q.lora_b.weight", np.zeros((4, 64)))])
    (tmp_path / "corrupted_dims.bin").write_bytes(raw)
    hdr, got = ga.lora_load(tmp_path / "corrupted_dims.bin")
    assert hdr["tensor_count"] == 2 and [a.shape for _, a in got] == [(32, 4), (4, 64)]


@pytest.mark.parametrize("case", ["magic", "version", "negative_count", "alpha_zero", "alpha_nan",
                                  "zero_dim", "huge_dims", "truncated_payload", "truncated_name",
                                  "missing"])
def test_malformed_files_are_rejected(tmp_path, case):
    a = np.ones((4, 2), np.float32)
    good = _record("blk.0.attn_q.lora_a.weight", a)
    raw = {
        "magic": _file(1, 2, 4.0, [good], magic=0x12345678),
        "version": _file(1, 2, 4.0, [good], version=2),
        "negative_count": _file(1, 2, 4.0, [], count=-1),
        "alpha_zero": _file(1, 2, 0.0, [good]),
        "alpha_nan": _file(1, 2, float("nan"), [good]),
        "zero_dim": _file(1, 2, 4.0, [_dotnet_string("blk.0.x.lora_a.weight") + struct.pack("<ii", 0, 2)]),
        # (2^31 - 1)^2 floats: the payload size overflows 63 bits
        "huge_dims": _file(1, 2, 4.0, [_dotnet_string("blk.0.x.lora_a.weight")
                                       + struct.pack("<ii", 2**31 - 1, 2**31 - 1) + a.tobytes()]),
        "truncated_payload": _file(1, 2, 4.0, [good[:-4]]),
        "truncated_name": _file(1, 2, 4.0, [_dotnet_string("blk.0.attn_q.lora_a.weight")[:10]]),
    }.get(case)
    p = tmp_path / "bad.bin"
    if raw is not None:
        p.write_bytes(raw)
    with pytest.raises(ga.InvalidData) as e:
        ga.lora_load(p)
    assert e.value.code == ga.ERR_DATA


def test_rank_zero_allows_any_alpha_and_bad_calls_are_rejected(tmp_path):
    (tmp_path / "r0.bin").write_bytes(_file(1, 0, 0.0, []))
    hdr, got = ga.lora_load(tmp_path / "r0.bin")
    assert hdr["rank"] == 0 and got == []
    with pytest.raises(ga.InvalidArgument):
        ga.lora_save(tmp_path / "x.bin", 1, 2, 4.0, [("a", np.zeros((0, 2), np.float32))])


def _reader(path):
    import ctypes

    L = ga.load()
    hdr = ga.LoraHeader()
    r = ctypes.c_void_p()
    assert L.glacier_lora_open(os.fsencode(path), ctypes.byref(hdr), ctypes.byref(r)) == ga.OK
    return L, r


def test_retry_after_a_too_small_name_buffer_reads_the_same_record(tmp_path):
    """A name buffer that is too small leaves the reader at the record's start:
    the retry the error text invites reads the record, and the rest follows."""
    import ctypes

    ts = _tensors(seed=4)
    long_name = "blk.0." + "x" * 300 + ".lora_a.weight"  # two-byte length prefix
    ts[0] = (long_name, ts[0][1])
    path = tmp_path / "adapter_model.bin"
    ga.lora_save(path, 1, 4, 8.0, ts)
    L, r = _reader(path)
    try:
        d0, d1 = ctypes.c_int32(), ctypes.c_int32()
        small = ctypes.create_string_buffer(16)
        rc = L.glacier_lora_next(r, small, len(small), ctypes.byref(d0), ctypes.byref(d1))
        assert rc == ga.ERR_INVALID_ARGUMENT
        need = int(L.glacier_attn_last_error().decode().rsplit("needs ", 1)[1].split()[0])
        assert need == len(long_name) + 1
        for name, want in ts:
            buf = ctypes.create_string_buffer(need)
            assert L.glacier_lora_next(r, buf, need, ctypes.byref(d0), ctypes.byref(d1)) == ga.OK
            assert buf.value.decode() == name and (d0.value, d1.value) == want.shape
            got = np.empty(want.shape, np.float32)
            assert L.glacier_lora_read(r, got.ctypes.data_as(ctypes.c_void_p), 0) == ga.OK
            np.testing.assert_array_equal(got, want)
    finally:
        L.glacier_lora_close(r)


@pytest.mark.parametrize("cut", ["name", "dims", "payload"])
def test_a_malformed_record_fails_every_later_call(tmp_path, cut):
    """After a truncated or malformed record the reader stays failed: no later
    call reads the rest of the (untrusted) bytes as new records."""
    import ctypes

    ts = _tensors(seed=5)
    raw = _file(1, 4, 8.0, [_record(n, a) for n, a in ts])
    first = len(_file(1, 4, 8.0, [])) + len(_record(*ts[0]))
    name_len = len(_dotnet_string(ts[1][0]))
    end = {"name": first + 3, "dims": first + name_len + 2, "payload": first + name_len + 8 + 5}[cut]
    path = tmp_path / "adapter_model.bin"
    path.write_bytes(raw[:end])
    L, r = _reader(path)
    try:
        d0, d1 = ctypes.c_int32(), ctypes.c_int32()
        buf = ctypes.create_string_buffer(256)
        assert L.glacier_lora_next(r, buf, 256, ctypes.byref(d0), ctypes.byref(d1)) == ga.OK
        assert L.glacier_lora_read(r, None, 0) == ga.OK
        assert L.glacier_lora_next(r, buf, 256, ctypes.byref(d0), ctypes.byref(d1)) == ga.ERR_DATA
        for _ in range(2):
            assert L.glacier_lora_next(r, buf, 256, ctypes.byref(d0), ctypes.byref(d1)) == ga.ERR_DATA
            assert L.glacier_lora_read(r, None, 0) == ga.ERR_DATA
    finally:
        L.glacier_lora_close(r)
