"""The lmio checkpoint format (ai/optim/lmio.lua) through the C ABI's host-side
save/load (no device involved, so these run on the CPU).

The library's writer and reader are checked against an independent reader and
writer below, written from the format lmio.lua documents and implements
(lmio.lua:5-13 layout, :226-257 header, :259-313 tensors, :393-611 reading):
  "lanternl-checkpoint <v>\\n", a space-separated key=value header line,
  then per tensor "<rows> <cols>\\n" + raw little-endian values (bin) or
  "<rows> <cols>|v,v,...\\n" (text); v1 files have neither the tag line nor
  the "r c|" prefix.  Writer -> independent reader and independent writer ->
  reader are both bit-exact on fp32 data; keep_last rotation, refusals and
  error messages follow lmio.lua.
"""
import math
import os
import struct

import numpy as np
import pytest

from lanternl_amd import lmtrain
from lanternl_amd._lib import LanternlHipError

V, D, L, H, F, T = 37, 12, 2, 3, 20, 9


def _cfg(**kw):
    a = dict(vocab=V, dim=D, layers=L, heads=H, ffn=F, batch=2, seq=T)
    a.update(kw)
    return lmtrain.config(**a)


def _params(cfg, seed=0):
    rng = np.random.default_rng(seed)
    return rng.standard_normal(lmtrain.num_params(cfg)).astype(np.float32)


def _shapes(cfg):
    return [(r, c) for (_, _, r, c) in lmtrain.param_table(cfg)]


# ---------------------------------------------------------------- independent format code
def _read_lmio(path):
    with open(path, "rb") as f:
        data = f.read()
    pos = 0

    def line():
        nonlocal pos
        e = data.index(b"\n", pos)
        s = data[pos:e].decode()
        pos = e + 1
        return s.rstrip("\r")

    l1 = line()
    if l1.startswith("lanternl-checkpoint"):
        version = int(l1.split()[1])
        header = line()
    else:
        version, header = 1, l1
    kv = dict(tok.split("=", 1) for tok in header.split() if "=" in tok)
    fmt = kv.get("format", "text")
    es = 4 if kv.get("dtype", "f64") == "f32" else 8
    n = int(kv["nparams"]) if "nparams" in kv else 2 + 9 * int(kv["layers"])
    tensors = []
    for _ in range(n):
        if fmt == "bin":
            r, c = map(int, line().split())
            raw = data[pos:pos + r * c * es]
            pos += r * c * es
            vals = np.frombuffer(raw, dtype="<f4" if es == 4 else "<f8").astype(np.float64)
        else:
            s = line()
            if version >= 2:
                rc, body = s.split("|", 1)
                r, c = map(int, rc.split())
            else:
                body, r, c = s, None, None
            vals = np.array([float(x) for x in body.split(",") if x], dtype=np.float64)
        tensors.append((r, c, vals))
    assert pos == len(data), "trailing bytes"
    return version, kv, tensors


def _write_lmio(path, cfg, params, version=3, fmt="bin", dtype="f32", crlf=False, fields=None):
    eol = "\r\n" if crlf else "\n"
    hdr = (f"format={fmt} dtype={dtype} endian=le vocab={cfg.vocab} dim={cfg.dim} layers={cfg.layers} "
           f"heads={cfg.heads} ffn={cfg.ffn}")
    if version >= 3:
        hdr += f" pos=rope causal=1 tie=1 max_seq={cfg.seq} rope_base=10000 nparams={2 + 9 * cfg.layers}"
        hdr += " backend=cpu epoch=4 loss=2.5 best_loss=2.25"
    if fields:
        hdr += " " + fields
    out = b""
    if version >= 2:
        out += f"lanternl-checkpoint {version}{eol}".encode()
    out += (hdr + eol).encode()
    off = 0
    for (r, c) in _shapes(cfg):
        vals = params[off:off + r * c].astype(np.float64)
        off += r * c
        if fmt == "bin":
            out += f"{r} {c}{eol}".encode()
            out += vals.astype("<f4" if dtype == "f32" else "<f8").tobytes()
        else:
            body = ",".join(repr(float(v)) if math.isfinite(v) else ("nan" if v != v else ("inf" if v > 0 else "-inf"))
                            for v in vals)
            out += ((f"{r} {c}|" if version >= 2 else "") + body + eol).encode()
    with open(path, "wb") as f:
        f.write(out)


# ---------------------------------------------------------------- writer -> independent reader
@pytest.mark.parametrize("fmt", ["bin", "text"])
def test_save_matches_lmio_layout(tmp_path, fmt):
    cfg = _cfg()
    p = _params(cfg, 1)
    path = tmp_path / "model.ckpt"
    lmtrain.save_checkpoint(path, cfg, p, fmt=fmt, epoch=7, loss=3.25, best_loss=float("inf"), extra="note=x")
    version, kv, tensors = _read_lmio(path)
    assert version == 3
    assert kv["format"] == fmt and kv["dtype"] == "f32" and kv["endian"] == "le"
    assert (kv["vocab"], kv["dim"], kv["layers"], kv["heads"], kv["ffn"]) == tuple(map(str, (V, D, L, H, F)))
    assert kv["pos"] == "rope" and kv["tie"] == "1" and kv["causal"] == "1"
    assert kv["max_seq"] == str(T) and float(kv["rope_base"]) == 10000.0
    assert kv["nparams"] == str(2 + 9 * L) and kv["backend"] == "luatl_adapter"
    assert kv["epoch"] == "7" and kv["loss"] == "3.25" and kv["best_loss"] == "nan" and kv["note"] == "x"
    assert [(r, c) for (r, c, _) in tensors] == _shapes(cfg)
    got = np.concatenate([t[2] for t in tensors])
    assert np.array_equal(got.astype(np.float32), p)      # %.9g round-trips fp32 exactly
    assert not [n for n in os.listdir(tmp_path) if ".tmp" in n]


# ---------------------------------------------------------------- independent writer -> reader
@pytest.mark.parametrize("version,fmt,dtype,crlf", [(3, "bin", "f32", False), (3, "bin", "f64", False),
                                                    (3, "text", "f32", False), (2, "text", "f32", True),
                                                    (1, "text", "f64", False)])
def test_load_every_lmio_version(tmp_path, version, fmt, dtype, crlf):
    cfg = _cfg()
    p = _params(cfg, 2)
    path = tmp_path / "in.ckpt"
    _write_lmio(path, cfg, p, version, fmt, dtype, crlf)
    got, hdr = lmtrain.load_checkpoint(path, cfg)
    assert np.array_equal(got, p)
    assert hdr["version"] == version and hdr["format"] == fmt and hdr["dtype"] == dtype
    if version >= 3:
        assert hdr["epoch"] == 4 and hdr["loss"] == 2.5 and hdr["best_loss"] == 2.25 and hdr["max_seq"] == T
    else:
        assert hdr["epoch"] == -1 and math.isnan(hdr["loss"])


def test_round_trip_and_special_values(tmp_path):
    cfg = _cfg()
    p = _params(cfg, 3)
    p[0], p[5], p[17] = np.nan, np.inf, -np.inf
    for fmt in ("bin", "text"):
        path = tmp_path / f"rt.{fmt}"
        lmtrain.save_checkpoint(path, cfg, p, fmt=fmt)
        got, _ = lmtrain.load_checkpoint(path, cfg)
        assert np.isnan(got[0]) and got[5] == np.inf and got[17] == -np.inf
        mask = np.isfinite(p)
        assert np.array_equal(got[mask], p[mask])


def test_keep_last_rotation(tmp_path):
    """lmio.lua:127-135: with keep = K the older files shift to path.1 .. path.(K-1)."""
    cfg = _cfg()
    path = tmp_path / "run.ckpt"
    for epoch in range(1, 5):
        lmtrain.save_checkpoint(path, cfg, _params(cfg, epoch), epoch=epoch, keep=3)
    names = sorted(os.listdir(tmp_path))
    assert names == ["run.ckpt", "run.ckpt.1", "run.ckpt.2"]
    for name, epoch in (("run.ckpt", 4), ("run.ckpt.1", 3), ("run.ckpt.2", 2)):
        got, hdr = lmtrain.load_checkpoint(tmp_path / name, cfg)
        assert hdr["epoch"] == epoch and np.array_equal(got, _params(cfg, epoch))


def _expect_error(fn, code_text):
    with pytest.raises(LanternlHipError) as e:
        fn()
    assert code_text in str(e.value)


def test_refusals(tmp_path):
    cfg = _cfg()
    p = _params(cfg, 4)
    path = tmp_path / "x.ckpt"
    lmtrain.save_checkpoint(path, cfg, p)
    # another model size (lmio.lua:549-555 per-tensor shape; header sizes first)
    _expect_error(lambda: lmtrain.load_checkpoint(path, _cfg(dim=16, heads=4)), "dim=12")
    # truncated inside a tensor
    data = path.read_bytes()
    (tmp_path / "t.ckpt").write_bytes(data[:-10])
    _expect_error(lambda: lmtrain.load_checkpoint(tmp_path / "t.ckpt", cfg), "truncated inside parameter")
    # a newer version, an untied head, another tensor count
    _write_lmio(tmp_path / "v4.ckpt", cfg, p, version=3)
    b = (tmp_path / "v4.ckpt").read_bytes().replace(b"lanternl-checkpoint 3", b"lanternl-checkpoint 4", 1)
    (tmp_path / "v4.ckpt").write_bytes(b)
    _expect_error(lambda: lmtrain.load_checkpoint(tmp_path / "v4.ckpt", cfg), "format v4")
    _write_lmio(tmp_path / "tie.ckpt", cfg, p, fields="")
    b = (tmp_path / "tie.ckpt").read_bytes().replace(b"tie=1", b"tie=0", 1)
    (tmp_path / "tie.ckpt").write_bytes(b)
    _expect_error(lambda: lmtrain.load_checkpoint(tmp_path / "tie.ckpt", cfg), "tie=0")
    b = (tmp_path / "tie.ckpt").read_bytes().replace(b"tie=0", b"tie=1").replace(
        f"nparams={2 + 9 * L}".encode(), b"nparams=5", 1)
    (tmp_path / "np.ckpt").write_bytes(b)
    _expect_error(lambda: lmtrain.load_checkpoint(tmp_path / "np.ckpt", cfg), "5 parameter tensors")
    # a value that is not a number (text)
    _write_lmio(tmp_path / "bad.ckpt", cfg, p, fmt="text")
    b = (tmp_path / "bad.ckpt").read_bytes()
    i = b.index(b"|") + 1
    (tmp_path / "bad.ckpt").write_bytes(b[:i] + b"abc" + b[b.index(b",", i):])
    _expect_error(lambda: lmtrain.load_checkpoint(tmp_path / "bad.ckpt", cfg), "is not a number ('abc')")
    # missing file, empty file
    _expect_error(lambda: lmtrain.load_checkpoint(tmp_path / "none.ckpt", cfg), "cannot open")
    (tmp_path / "empty.ckpt").write_bytes(b"")
    _expect_error(lambda: lmtrain.load_checkpoint(tmp_path / "empty.ckpt", cfg), "is empty")
    # a write into a directory that does not exist leaves nothing behind
    _expect_error(lambda: lmtrain.save_checkpoint(tmp_path / "no" / "x.ckpt", cfg, p), "cannot write")


def test_bin_values_are_little_endian_fp32(tmp_path):
    cfg = _cfg()
    p = np.arange(lmtrain.num_params(cfg), dtype=np.float32) * np.float32(0.5)
    path = tmp_path / "le.ckpt"
    lmtrain.save_checkpoint(path, cfg, p)
    data = path.read_bytes()
    first = data.index(b"\n", data.index(b"\n") + 1) + 1          # after the two header lines
    nl = data.index(b"\n", first)
    assert data[first:nl] == f"{V} {D}".encode()
    assert struct.unpack("<3f", data[nl + 1:nl + 13]) == (0.0, 0.5, 1.0)
