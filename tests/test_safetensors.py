"""The safetensors loader's header checks, on the CPU.

quicklm_amd/csrc/host/safetensors.cpp maps a file and validates every
tensor's entry before any byte is read or uploaded (the reference's loader,
src/io/safetensors.cpp:121-246, trusts the header). A tensor must lie inside
the file and hold exactly prod(shape) x element-size bytes, with no negative
dimension: the device upload copies `nbytes` while the quantiser reads by
shape, so any mismatch would read or write past a buffer.
"""

import ctypes as C
import json
import os
import struct
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOST = os.path.join(ROOT, "quicklm_amd", "csrc", "host")


@pytest.fixture(scope="module")
def st(tmp_path_factory):
    d = tmp_path_factory.mktemp("stprobe")
    so = str(d / "libstprobe.so")
    subprocess.run(["g++", "-std=c++17", "-O1", "-shared", "-fPIC", "-Wall", "-I", HOST,
                    os.path.join(ROOT, "tests", "st_probe.cpp"),
                    os.path.join(HOST, "safetensors.cpp"), "-o", so], check=True)
    return C.CDLL(so)


def write(path, header, data_len):
    hj = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hj)))
        f.write(hj)
        f.write(b"\0" * data_len)


def open_file(st, path):
    err = C.create_string_buffer(512)
    rc = st.st_open(str(path).encode(), err, 512)
    return rc, err.value.decode()


def test_valid_header_accepted(st, tmp_path):
    p = tmp_path / "ok.safetensors"
    write(p, {"a": {"dtype": "F32", "shape": [2, 3], "data_offsets": [0, 24]},
              "b": {"dtype": "BF16", "shape": [4], "data_offsets": [24, 32]},
              "__metadata__": {"format": "pt"}}, 32)
    assert open_file(st, p) == (2, "")


@pytest.mark.parametrize("entry,msg", [
    ({"dtype": "F32", "shape": [2, 3], "data_offsets": [0, 28]}, "needs 24"),   # range too large
    ({"dtype": "F32", "shape": [2, 3], "data_offsets": [0, 20]}, "needs 24"),   # range too small
    ({"dtype": "BF16", "shape": [2, 3], "data_offsets": [0, 24]}, "needs 12"),  # dtype mismatch
    ({"dtype": "F32", "shape": [-2, 3], "data_offsets": [0, 24]}, "bad shape"),
    ({"dtype": "F32", "shape": [2.5, 3], "data_offsets": [0, 24]}, "bad shape"),
    ({"dtype": "F32", "shape": [2, 3], "data_offsets": [8, 32]}, "out of file bounds"),
    ({"dtype": "F32", "shape": [2, 3], "data_offsets": [24, 0]}, "out of file bounds"),
    ({"dtype": "F32", "shape": [2, 3], "data_offsets": [-8, 16]}, "out of file bounds"),
    ({"dtype": "F32", "shape": [1 << 40, 1 << 40], "data_offsets": [0, 24]}, "too large"),
])
def test_bad_entry_rejected(st, tmp_path, entry, msg):
    p = tmp_path / "bad.safetensors"
    write(p, {"t": entry}, 28)
    rc, err = open_file(st, p)
    assert rc == -1 and msg in err, err
