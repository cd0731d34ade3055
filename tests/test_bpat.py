"""bpat files (fused_gpu::io, crates/fused_gpu/src/io/*): the C++ reader and
writer checked against an independent restatement of the layouts in
io/headers.rs:1-117 (struct + zlib.crc32), against the reference's own file
data/v2f32_readme.bpat (stored compressed under tests/golden/), and for
every header by round trips.  No device is needed: files are written from
host memory (fg_bpat_save_host) and parsed into host memory."""
import lzma
import os
import struct
import zlib

import numpy as np
import pytest
import torch

from conftest import GOLDEN

from ferrograd_amd import io as fio
from ferrograd_amd._lib import FgError

H = fio.BpatHeader
MAGIC = {H.BpatV0: b"bpat", H.BpatV1: b"BPATv1\0\0", H.BpatV1M: b"BPATv1m\0",
         H.BpatV2f16: b"BPAT\0f16", H.BpatV2bf16: b"BPATbf16", H.BpatV2f32: b"BPAT\0f32"}
DIM = {H.BpatV0: 8, H.BpatV1: 8, H.BpatV1M: 4, H.BpatV2f16: 4, H.BpatV2bf16: 4, H.BpatV2f32: 4}
CRC = {H.BpatV1, H.BpatV1M}


def bf16_words(x):
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def encode(header, arrays):
    """Independent writer: the layout of io/headers.rs with zlib's CRC-32."""
    out = bytearray(MAGIC[header]) + bytes([len(arrays)])
    d = "<Q" if DIM[header] == 8 else "<I"
    for a in arrays:
        a = np.asarray(a, dtype=np.float32)
        start = len(out)
        out += struct.pack(d, a.ndim)
        for n in a.shape:
            out += struct.pack(d, n)
        if header in (H.BpatV0, H.BpatV1):
            out += a.astype("<f8").tobytes()
        elif header in (H.BpatV1M, H.BpatV2f32):
            out += a.astype("<f4").tobytes()
        elif header == H.BpatV2f16:
            out += a.astype("<f2").tobytes()
        else:
            out += bf16_words(a).astype("<u2").tobytes()
        if header in CRC:
            out += struct.pack("<I", zlib.crc32(bytes(out[start:])))
    if header in CRC:
        out += struct.pack("<I", zlib.crc32(bytes(out)))
    return bytes(out)


@pytest.fixture(scope="module")
def readme_bytes():
    with lzma.open(os.path.join(GOLDEN, "v2f32_readme.bpat.xz"), "rb") as f:
        return f.read()


def test_reference_file_parses_and_rewrites_byte_identical(readme_bytes, tmp_path):
    """The reference's own file (5 fp32 tensors written by its V2 f32
    writer): shapes and values match an independent parse, and writing the
    values back reproduces the file byte for byte."""
    p = tmp_path / "readme.bpat"
    p.write_bytes(readme_bytes)
    # Independent parse.
    b, off = readme_bytes, 9
    assert b[:8] == MAGIC[H.BpatV2f32] and b[8] == 5
    arrays = []
    for _ in range(b[8]):
        rank = struct.unpack_from("<I", b, off)[0]
        shape = struct.unpack_from(f"<{rank}I", b, off + 4)
        off += 4 + 4 * rank
        n = int(np.prod(shape))
        arrays.append(np.frombuffer(b, "<f4", n, off).reshape(shape))
        off += 4 * n
    assert off == len(b)
    with fio.BpatFile(p) as f:
        assert (f.header, f.count) == (H.BpatV2f32, 5)
        for i, a in enumerate(arrays):
            assert f.shape(i) == a.shape
            assert np.array_equal(f.read_f32(i), a)
        back = [f.read_f32(i) for i in range(f.count)]
    q = tmp_path / "rewrite.bpat"
    fio.save_arrays(q, back, H.BpatV2f32)
    assert q.read_bytes() == readme_bytes


@pytest.mark.parametrize("header", [H.BpatV0, H.BpatV1, H.BpatV1M, H.BpatV2f16, H.BpatV2bf16,
                                    H.BpatV2f32])
def test_writer_matches_independent_encoding(header, tmp_path):
    rng = np.random.default_rng(header)
    arrays = [rng.standard_normal((7, 5)).astype(np.float32),
              rng.standard_normal((3,)).astype(np.float32),
              np.zeros((0, 4), np.float32),
              (1e-6 * rng.standard_normal((2, 3, 4))).astype(np.float32)]
    p = tmp_path / "t.bpat"
    fio.save_arrays(p, arrays, header)
    assert p.read_bytes() == encode(header, arrays)
    with fio.BpatFile(p) as f:
        assert f.header == header and f.count == len(arrays)
        for i, a in enumerate(arrays):
            assert f.shape(i) == a.shape
            got = f.read_f32(i)
            if header == H.BpatV2f16:
                want = a.astype(np.float16).astype(np.float32)
            elif header == H.BpatV2bf16:
                want = (bf16_words(a).astype(np.uint32) << 16).view(np.float32).reshape(a.shape)
            else:
                want = a
            assert np.array_equal(got, want)


def test_16bit_arrays_are_written_without_conversion(tmp_path):
    a16 = np.arange(-8, 8, dtype=np.float32).astype(np.float16).reshape(4, 4)
    b16 = bf16_words(np.linspace(-3, 3, 10, dtype=np.float32))
    p = tmp_path / "h.bpat"
    fio.save_arrays(p, [a16], H.BpatV2f16)
    assert p.read_bytes() == encode(H.BpatV2f16, [a16.astype(np.float32)])
    fio.save_arrays(p, [b16], H.BpatV2bf16)
    with fio.BpatFile(p) as f:
        got = f.read_f32(0)
    assert np.array_equal(got, (b16.astype(np.uint32) << 16).view(np.float32))


def test_corrupt_files_are_rejected(tmp_path):
    arrays = [np.ones((4, 4), np.float32), np.arange(6, dtype=np.float32)]
    good = encode(H.BpatV1M, arrays)
    cases = {
        "magic": b"XXXX" + good[4:],
        "tensor_crc": good[:-9] + bytes([good[-9] ^ 1]) + good[-8:],
        "data": good[:20] + bytes([good[20] ^ 0x80]) + good[21:],
        "file_crc": good[:-1] + bytes([good[-1] ^ 1]),
        "truncated": good[:-6],
        "trailing": good + b"\0",
    }
    for name, blob in cases.items():
        p = tmp_path / f"{name}.bpat"
        p.write_bytes(blob)
        with pytest.raises(FgError) as e:
            fio.BpatFile(p)
        assert e.value.code == 10, name  # SERIALIZATION
    with pytest.raises(FgError) as e:
        fio.BpatFile(tmp_path / "missing.bpat")
    assert e.value.code == 11  # FILE_NOT_FOUND
    p = tmp_path / "ok.bpat"
    p.write_bytes(good)
    with fio.BpatFile(p) as f:
        assert f.count == 2 and np.array_equal(f.read_f32(1), arrays[1])
