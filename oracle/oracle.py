"""numpy front end of the C oracle (``oracle/relm_mp_oracle.c``).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of bench.py as the checker.  The product package
(``relmo_amd``) never imports it.

Each wrapper restates one reference CPU routine (see the C file for the
file:line of relmo's ``src/_ops/mp/mp_ops.cpp`` it follows) and raises the
reference's error for an index out of range: ``OracleIndexError`` with the
loop message of the sum and copy ops, and for the logsumexp ops (ATen call
sequences there) ATen's errors in call order - ``IndexError`` from
index_select, ``OracleIndexError`` with ATen's message from scatter_reduce_ /
index_add_.

Parity status of each function (how it is pinned, see tests/test_oracle.py):
  fanout_scatter                  pinned: reference library (oracle/_ref) bit-exact,
                                  golden fixtures, brute-force numpy loop
  fanout_scatter_backward         pinned: reference library bit-exact, golden
                                  fixtures, conservation / linearity, float64 truth
  fanin_reduce_sum                pinned: reference library bit-exact, golden
                                  fixtures, conservation / linearity, float64 truth
  fanin_reduce_sum_backward       pinned: reference library bit-exact, golden fixtures
  fanin_reduce_logsumexp          pinned: reference library (rtol 1e-6), closed forms
                                  (single message, n equal values, empty row,
                                  shift invariance, max <= lse <= max + log n)
  fanin_reduce_logsumexp_backward pinned: reference library (rtol 1e-6), softmax
                                  weights sum to one, float64 finite differences
  csr_build / inverse_build       pinned: numpy stable argsort / bincount, brute force
  fanout_into_slots /             compositions of the two fanout functions above
  fanout_backward_from_slots      with numpy's row-major reshape (the models' input
                                  assembly); pinned through them and a per-element loop
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle_relm_mp.so"
SOURCE = HERE / "relm_mp_oracle.c"


class OracleIndexError(RuntimeError):
    """Index out of range, with the reference's message."""


class _Bad(ctypes.Structure):
    _fields_ = [
        ("which", ctypes.c_int32),
        ("pad", ctypes.c_int32),
        ("edge", ctypes.c_int64),
        ("value", ctypes.c_int64),
        ("bound", ctypes.c_int64),
    ]


_LIB: ctypes.CDLL | None = None


def build() -> Path:
    """Compile the oracle if its library is missing or older than the source."""

    if not LIB_PATH.exists() or LIB_PATH.stat().st_mtime < SOURCE.stat().st_mtime:
        subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        build()
        _LIB = ctypes.CDLL(str(LIB_PATH))
    return _LIB


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def _idx(a) -> np.ndarray:
    a = np.ascontiguousarray(np.asarray(a, dtype=np.int64))
    assert a.ndim == 1
    return a


def _vals(a) -> np.ndarray:
    a = np.ascontiguousarray(np.asarray(a))
    assert a.dtype in (np.float32, np.float64) and a.ndim == 2, a.dtype
    return a


def _suffix(a: np.ndarray) -> str:
    return "f32" if a.dtype == np.float32 else "f64"


def _raise(rc: int, bad: _Bad, names: tuple[str, str]) -> None:
    if rc == 0:
        return
    if rc == 2:
        raise OracleIndexError(
            f"{names[bad.which]} index out of bounds: {bad.value} not in [0, {bad.bound})."
        )
    raise MemoryError("oracle allocation failed")


def fanout_scatter(x_cat, src_global_idx, flat_dst, out_rows: int) -> np.ndarray:
    """mp_ops.cpp:2815-2836."""

    x = _vals(x_cat)
    src, dst = _idx(src_global_idx), _idx(flat_dst)
    out = np.empty((int(out_rows), x.shape[1]), dtype=x.dtype)
    bad = _Bad()
    fn = getattr(lib(), "oracle_fanout_scatter_" + _suffix(x))
    rc = fn(_p(x), ctypes.c_int64(x.shape[0]), ctypes.c_int64(x.shape[1]), _p(src), _p(dst),
            ctypes.c_int64(src.size), ctypes.c_int64(out.shape[0]), _p(out), ctypes.byref(bad))
    _raise(rc, bad, ("src_global_idx", "flat_dst"))
    return out


def fanout_scatter_backward(grad_out, src_global_idx, flat_dst, x_rows: int) -> np.ndarray:
    """mp_ops.cpp:2838-2861."""

    g = _vals(grad_out)
    src, dst = _idx(src_global_idx), _idx(flat_dst)
    out = np.empty((int(x_rows), g.shape[1]), dtype=g.dtype)
    bad = _Bad()
    fn = getattr(lib(), "oracle_fanout_scatter_backward_" + _suffix(g))
    rc = fn(_p(g), ctypes.c_int64(g.shape[0]), ctypes.c_int64(g.shape[1]), _p(src), _p(dst),
            ctypes.c_int64(src.size), ctypes.c_int64(out.shape[0]), _p(out), ctypes.byref(bad))
    _raise(rc, bad, ("src_global_idx", "flat_dst"))
    return out


def fanout_into_slots(x_cat, src_global_idx, flat_dst, out, col_offset: int, slots: int) -> np.ndarray:
    """The central input assembly of relmo/models/hetero_mp/fused.py:299-375:
    fanout_scatter into [lines * slots, D] rows, reshaped to [lines, slots * D]
    and copied into columns [col_offset, col_offset + slots * D) of a copy of
    ``out``; the other columns keep their values."""

    x = _vals(x_cat)
    res = np.array(out, copy=True)
    lines, d = res.shape[0], x.shape[1]
    rows = fanout_scatter(x, src_global_idx, flat_dst, lines * slots)
    res[:, col_offset:col_offset + slots * d] = rows.reshape(lines, slots * d)
    return res


def fanout_backward_from_slots(grad, src_global_idx, flat_dst, x_rows: int, col_offset: int,
                               slots: int, emb: int) -> np.ndarray:
    """Backward of ``fanout_into_slots``: fanout_scatter_backward of the
    argument columns of ``grad`` read as [lines * slots, emb] rows."""

    g = _vals(grad)
    rows = np.ascontiguousarray(g[:, col_offset:col_offset + slots * emb]).reshape(-1, emb)
    return fanout_scatter_backward(rows, src_global_idx, flat_dst, x_rows)


def fanin_reduce_sum(rel_flat, flat_src, dst_idx, dim_size: int) -> np.ndarray:
    """mp_ops.cpp:2863-2886."""

    r = _vals(rel_flat)
    src, dst = _idx(flat_src), _idx(dst_idx)
    out = np.empty((int(dim_size), r.shape[1]), dtype=r.dtype)
    bad = _Bad()
    fn = getattr(lib(), "oracle_fanin_reduce_sum_" + _suffix(r))
    rc = fn(_p(r), ctypes.c_int64(r.shape[0]), ctypes.c_int64(r.shape[1]), _p(src), _p(dst),
            ctypes.c_int64(src.size), ctypes.c_int64(out.shape[0]), _p(out), ctypes.byref(bad))
    _raise(rc, bad, ("flat_src", "dst_idx"))
    return out


def _outside(idx: np.ndarray, size: int) -> np.ndarray:
    return (idx < 0) | (idx >= size)


def _aten_index_select_check(idx: np.ndarray, rows: int) -> None:
    """ATen's index_select on the CPU: IndexError for any index outside the rows."""

    if np.any(_outside(idx, rows)):
        raise IndexError("index out of range in self")


def _aten_scatter_check(idx: np.ndarray, size: int) -> None:
    """ATen's scatter_reduce_ / index_add_ on the CPU: the first index outside
    [0, size) in edge order."""

    bad = np.flatnonzero(_outside(idx, size))
    if bad.size:
        raise OracleIndexError(f"index {int(idx[bad[0]])} is out of bounds for dimension 0 with size {size}")


def fanin_reduce_logsumexp(rel_flat, flat_src, dst_idx, dim_size: int) -> np.ndarray:
    """mp_ops.cpp:3019-3035 (the CPU ATen sequence, restated with libm exp/log).
    An index out of range raises ATen's error of the call that meets it first:
    index_select over flat_src, then scatter_reduce_ over dst_idx."""

    r = _vals(rel_flat)
    src, dst = _idx(flat_src), _idx(dst_idx)
    if src.size and dim_size and r.shape[1]:
        _aten_index_select_check(src, r.shape[0])
        _aten_scatter_check(dst, int(dim_size))
    out = np.empty((int(dim_size), r.shape[1]), dtype=r.dtype)
    bad = _Bad()
    fn = getattr(lib(), "oracle_fanin_reduce_logsumexp_" + _suffix(r))
    rc = fn(_p(r), ctypes.c_int64(r.shape[0]), ctypes.c_int64(r.shape[1]), _p(src), _p(dst),
            ctypes.c_int64(src.size), ctypes.c_int64(out.shape[0]), _p(out), ctypes.byref(bad))
    _raise(rc, bad, ("flat_src", "dst_idx"))
    return out


def fanin_reduce(rel_flat, flat_src, dst_idx, dim_size: int, mode: int) -> np.ndarray:
    """mp_ops.cpp:3327-3348 mode router."""

    if mode == 0:
        return fanin_reduce_sum(rel_flat, flat_src, dst_idx, dim_size)
    if mode == 1:
        return fanin_reduce_logsumexp(rel_flat, flat_src, dst_idx, dim_size)
    raise ValueError("Unsupported fanin_reduce mode. Supported: 0=sum, 1=logsumexp.")


def fanin_reduce_sum_backward(grad_out, flat_src, dst_idx, rel_rows: int) -> np.ndarray:
    """mp_ops.cpp:2888-2911."""

    g = _vals(grad_out)
    src, dst = _idx(flat_src), _idx(dst_idx)
    out = np.empty((int(rel_rows), g.shape[1]), dtype=g.dtype)
    bad = _Bad()
    fn = getattr(lib(), "oracle_fanin_reduce_sum_backward_" + _suffix(g))
    rc = fn(_p(g), ctypes.c_int64(g.shape[0]), ctypes.c_int64(g.shape[1]), _p(src), _p(dst),
            ctypes.c_int64(src.size), ctypes.c_int64(out.shape[0]), _p(out), ctypes.byref(bad))
    _raise(rc, bad, ("flat_src", "dst_idx"))
    return out


def fanin_reduce_logsumexp_backward(grad_out, rel_flat, flat_src, dst_idx, out, rel_rows: int) -> np.ndarray:
    """mp_ops.cpp:2981-3003 (ATen fallback sequence, edge order).  An index out
    of range raises ATen's error of the call that meets it first: index_select
    of rel_flat rows (flat_src), of out and grad_out rows (dst_idx), then
    index_add_ into the rel_rows gradient rows (flat_src)."""

    g, r, o = _vals(grad_out), _vals(rel_flat), _vals(out)
    src, dst = _idx(flat_src), _idx(dst_idx)
    if src.size and rel_rows and g.shape[1]:
        _aten_index_select_check(src, r.shape[0])
        _aten_index_select_check(dst, o.shape[0])
        _aten_index_select_check(dst, g.shape[0])
        _aten_scatter_check(src, int(rel_rows))
    res = np.empty((int(rel_rows), g.shape[1]), dtype=r.dtype)
    bad = _Bad()
    fn = getattr(lib(), "oracle_fanin_reduce_logsumexp_backward_" + _suffix(r))
    rc = fn(_p(g), ctypes.c_int64(g.shape[0]), ctypes.c_int64(g.shape[1]), _p(r),
            ctypes.c_int64(r.shape[0]), _p(src), _p(dst), ctypes.c_int64(src.size), _p(o),
            ctypes.c_int64(res.shape[0]), _p(res), ctypes.byref(bad))
    _raise(rc, bad, ("flat_src", "dst_idx"))
    return res


def segment_sum_truth(table, read_idx, write_idx, out_rows: int) -> tuple[np.ndarray, np.ndarray]:
    """float64 sum of fp32 rows (and the sum of |terms|) per written row."""

    t = np.ascontiguousarray(table, dtype=np.float32)
    r, w = _idx(read_idx), _idx(write_idx)
    s = np.empty((int(out_rows), t.shape[1]), dtype=np.float64)
    a = np.empty_like(s)
    lib().oracle_segment_sum_truth(_p(t), ctypes.c_int64(t.shape[1]), _p(r), _p(w),
                                   ctypes.c_int64(r.size), ctypes.c_int64(s.shape[0]), _p(s), _p(a))
    return s, a


def fanin_logsumexp_truth(rel_flat, flat_src, dst_idx, dim_size: int) -> np.ndarray:
    """float64 logsumexp of fp32 messages."""

    t = np.ascontiguousarray(rel_flat, dtype=np.float32)
    src, dst = _idx(flat_src), _idx(dst_idx)
    out = np.empty((int(dim_size), t.shape[1]), dtype=np.float64)
    lib().oracle_fanin_logsumexp_truth(_p(t), ctypes.c_int64(t.shape[1]), _p(src), _p(dst),
                                       ctypes.c_int64(src.size), ctypes.c_int64(out.shape[0]), _p(out))
    return out


def csr_build(keys, num_keys: int) -> tuple[np.ndarray, np.ndarray]:
    """Stable CSR: offsets [num_keys + 1] and edge ids in stable key order."""

    k = _idx(keys)
    offsets = np.empty(int(num_keys) + 1, dtype=np.int32)
    perm = np.empty(k.size, dtype=np.int32)
    bad = _Bad()
    rc = lib().oracle_csr_build(_p(k), ctypes.c_int64(k.size), ctypes.c_int64(num_keys),
                                _p(offsets), _p(perm), ctypes.byref(bad))
    _raise(rc, bad, ("keys", "keys"))
    return offsets, perm


def inverse_build(keys, num_keys: int) -> tuple[np.ndarray, int]:
    """inv[k] = largest edge with key k (or -1) and the collision count."""

    k = _idx(keys)
    inv = np.empty(int(num_keys), dtype=np.int32)
    lib().oracle_inverse_build.restype = ctypes.c_int64
    collisions = lib().oracle_inverse_build(_p(k), ctypes.c_int64(k.size), ctypes.c_int64(num_keys), _p(inv))
    return inv, int(collisions)
