"""ctypes binding of ``librelm_mp_hip.so`` (declared in ``include/relm_mp.h``).

Tensors are passed as raw device pointers; outputs and workspaces are
allocated with torch on the tensors' device and every call is enqueued on
torch's current stream.  torch is imported before the library is opened so
that the process uses torch's HIP runtime (both carry the soname
``libamdhip64.so.7``; loading ours first would map a second runtime).
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "librelm_mp_hip.so"

OK = 0
ERR_INVALID_ARGUMENT = 1
ERR_INDEX_OUT_OF_BOUNDS = 2
ERR_UNSUPPORTED_MODE = 3
ERR_WORKSPACE = 4
ERR_HIP = 5

F32 = 0
F64 = 1
PLAN_INVERSE = 1
PLAN_CSR = 2
PLAN_SNAPSHOT = 1  # inverse-plan build flag: keep a snapshot of the indices

EXPORTED_SYMBOLS = (
    "relm_mp_last_error",
    "relm_mp_build_info",
    "relm_mp_fanout_scatter_workspace_size",
    "relm_mp_fanout_scatter",
    "relm_mp_fanout_scatter_backward_workspace_size",
    "relm_mp_fanout_scatter_backward",
    "relm_mp_fanin_reduce_workspace_size",
    "relm_mp_fanin_reduce",
    "relm_mp_fanin_reduce_noalloc",
    "relm_mp_fanin_reduce_sum_backward_workspace_size",
    "relm_mp_fanin_reduce_sum_backward",
    "relm_mp_fanin_reduce_logsumexp_backward_workspace_size",
    "relm_mp_fanin_reduce_logsumexp_backward",
    "relm_mp_inv_plan_bytes",
    "relm_mp_inv_plan_build",
    "relm_mp_inv_plan_build_async",
    "relm_mp_plan_validate",
    "relm_mp_csr_plan_bytes",
    "relm_mp_csr_plan_scratch_bytes",
    "relm_mp_csr_plan_build",
    "relm_mp_csr_plan_build_async",
    "relm_mp_plan_read_counts",
    "relm_mp_plan_compute_scratch_bytes",
    "relm_mp_plan_gather_last",
    "relm_mp_plan_segment_reduce",
    "relm_mp_plan_logsumexp_backward",
    "relm_mp_plan_fanin_backward_by_dst",
    "relm_mp_plan_fanin_backward_by_src",
    "relm_mp_pack_index",
    "relm_mp_plan_match_workspace_size",
    "relm_mp_plan_match",
    "relm_mp_rows_scale",
    "relm_mp_plan_segment_sum_scaled",
    "relm_mp_plan_segment_sum_msgdiv",
    "relm_mp_plan_gather_last_grouped",
    "relm_mp_plan_segment_sum_grouped",
    "relm_mp_film_mish",
    "relm_mp_film_mish_blocks",
    "relm_mp_film_mish_backward",
)


class Plan(ctypes.Structure):
    """Mirror of ``struct relm_mp_plan``."""

    _fields_ = [
        ("kind", ctypes.c_int32),
        ("hub_threshold", ctypes.c_int32),
        ("chunk_size", ctypes.c_int32),
        ("gather_identity", ctypes.c_int32),
        ("num_keys", ctypes.c_int64),
        ("num_edges", ctypes.c_int64),
        ("num_gather", ctypes.c_int64),
        ("collisions", ctypes.c_int64),
        ("max_degree", ctypes.c_int64),
        ("num_hubs", ctypes.c_int64),
        ("num_chunks", ctypes.c_int64),
        ("num_multi_hubs", ctypes.c_int64),
        ("num_items", ctypes.c_int64),
        ("num_short", ctypes.c_int64),
        ("inv", ctypes.c_void_p),
        ("offsets", ctypes.c_void_p),
        ("gather_sorted", ctypes.c_void_p),
        ("hub_key", ctypes.c_void_p),
        ("hub_chunk_base", ctypes.c_void_p),
        ("chunk_hub", ctypes.c_void_p),
        ("multi_hubs", ctypes.c_void_p),
        ("item_first", ctypes.c_void_p),
        ("item_short", ctypes.c_void_p),
        ("short_off", ctypes.c_void_p),
        ("short_gather", ctypes.c_void_p),
        ("counts", ctypes.c_void_p),
        ("snap_keys", ctypes.c_void_p),
        ("snap_gathers", ctypes.c_void_p),
        ("snap_key_plain", ctypes.c_void_p),
        ("snap_gather_plain", ctypes.c_void_p),
    ]


class IndexPart(ctypes.Structure):
    """Mirror of ``struct relm_mp_index_part``."""

    _fields_ = [
        ("a", ctypes.c_void_p),
        ("b", ctypes.c_void_p),
        ("n", ctypes.c_int64),
        ("a_mul", ctypes.c_int64),
        ("a_add", ctypes.c_int64),
        ("b_mul", ctypes.c_int64),
        ("b_add", ctypes.c_int64),
    ]


_i64 = ctypes.c_int64
_int = ctypes.c_int
_sz = ctypes.c_size_t
_vp = ctypes.c_void_p
_cp = ctypes.c_char_p
_PP = ctypes.POINTER(Plan)

_SIGNATURES = {
    "relm_mp_last_error": (_cp, []),
    "relm_mp_build_info": (_cp, []),
    "relm_mp_fanout_scatter_workspace_size": (_sz, [_i64, _i64]),
    "relm_mp_fanout_scatter": (_int, [_int, _vp, _i64, _i64, _vp, _vp, _i64, _i64, _vp, _vp, _sz, _vp]),
    "relm_mp_fanout_scatter_backward_workspace_size": (_sz, [_i64, _i64, _i64, _int]),
    "relm_mp_fanout_scatter_backward": (_int, [_int, _vp, _i64, _i64, _vp, _vp, _i64, _i64, _vp, _vp, _sz, _vp]),
    "relm_mp_fanin_reduce_workspace_size": (_sz, [_i64, _i64, _i64, _int]),
    "relm_mp_fanin_reduce": (_int, [_int, _vp, _i64, _i64, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _sz, _vp]),
    "relm_mp_fanin_reduce_noalloc": (_int, [_int, _vp, _i64, _i64, _vp, _vp, _i64, _i64, _i64, _vp, _vp]),
    "relm_mp_fanin_reduce_sum_backward_workspace_size": (_sz, [_i64, _i64, _i64, _int]),
    "relm_mp_fanin_reduce_sum_backward": (_int, [_int, _vp, _i64, _i64, _vp, _vp, _i64, _i64, _vp, _vp, _sz, _vp]),
    "relm_mp_fanin_reduce_logsumexp_backward_workspace_size": (_sz, [_i64, _i64, _i64, _int]),
    "relm_mp_fanin_reduce_logsumexp_backward": (
        _int,
        [_int, _vp, _i64, _i64, _vp, _i64, _vp, _vp, _i64, _vp, _i64, _vp, _vp, _sz, _vp],
    ),
    "relm_mp_inv_plan_bytes": (_sz, [_i64, _i64, _int]),
    "relm_mp_inv_plan_build": (_int, [_vp, _i64, _cp, _vp, _i64, _cp, _int, _i64, _int, _vp, _sz, _PP, _vp]),
    "relm_mp_inv_plan_build_async": (
        _int, [_vp, _i64, _cp, _vp, _i64, _cp, _int, _i64, _int, _vp, _sz, _PP, _vp]),
    "relm_mp_plan_validate": (_int, [_PP]),
    "relm_mp_csr_plan_bytes": (_sz, [_i64, _i64]),
    "relm_mp_csr_plan_scratch_bytes": (_sz, [_i64, _i64]),
    "relm_mp_csr_plan_build": (
        _int,
        [_vp, _i64, _cp, _vp, _i64, _cp, _int, _i64, _vp, _sz, _vp, _sz, _PP, _vp],
    ),
    "relm_mp_csr_plan_build_async": (
        _int,
        [_vp, _i64, _cp, _vp, _i64, _cp, _int, _i64, _vp, _sz, _vp, _sz, _PP, _vp],
    ),
    "relm_mp_plan_read_counts": (_int, [_PP, _vp]),
    "relm_mp_plan_compute_scratch_bytes": (_sz, [_PP, _i64, _int, _i64]),
    "relm_mp_plan_gather_last": (_int, [_int, _PP, _vp, _vp, _i64, _vp, _vp]),
    "relm_mp_plan_segment_reduce": (_int, [_int, _PP, _vp, _vp, _i64, _i64, _vp, _vp, _sz, _vp]),
    "relm_mp_plan_logsumexp_backward": (_int, [_int, _PP, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _sz, _vp]),
    "relm_mp_plan_fanin_backward_by_dst": (_int, [_int, _PP, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _i64, _vp]),
    "relm_mp_plan_fanin_backward_by_src": (
        _int, [_int, _PP, _i64, _vp, _vp, _vp, _i64, _vp, _i64, _vp, _sz, _int, ctypes.POINTER(ctypes.c_int64),
               _vp]),
    "relm_mp_pack_index": (_int, [ctypes.POINTER(IndexPart), ctypes.c_int32, _vp, _vp, _vp]),
    "relm_mp_plan_match_workspace_size": (_sz, []),
    "relm_mp_rows_scale": (_int, [_int, _vp, _vp, _int, _vp, _vp, _vp, _i64, _i64, _vp, _vp]),
    "relm_mp_plan_segment_sum_scaled": (_int, [_int, _PP, _vp, _i64, _int, _vp, _vp, _vp, _vp, _sz, _vp]),
    "relm_mp_plan_segment_sum_msgdiv": (_int, [_int, _PP, _vp, _i64, _vp, _vp, _vp, _vp, _sz, _vp]),
    "relm_mp_plan_gather_last_grouped": (_int, [_int, _PP, _vp, _vp, _i64, _i64, _i64, _vp, _vp]),
    "relm_mp_plan_segment_sum_grouped": (
        _int, [_int, _PP, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _sz, _vp]),
    "relm_mp_film_mish": (_int, [_vp, _i64, _i64, _vp, ctypes.c_int32, _vp, _vp, _vp, _vp, _vp]),
    "relm_mp_film_mish_blocks": (_i64, [_vp, ctypes.c_int32]),
    "relm_mp_film_mish_backward": (
        _int, [_vp, _vp, _i64, _i64, _vp, ctypes.c_int32, _vp, _vp, _vp, _vp, _vp, _i64, _vp]),
    "relm_mp_plan_match": (
        _int,
        [_vp, _vp, _i64, ctypes.POINTER(_PP), ctypes.c_int32, ctypes.POINTER(ctypes.c_int32), _vp,
         _sz, _vp],
    ),
}

_LIB: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """Open the library once and declare every signature."""

    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(
                f"{LIB_PATH} is missing; build it with `python -m relmo_amd.csrc.build`."
            )
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _LIB = handle
    return _LIB


def last_error() -> str:
    return lib().relm_mp_last_error().decode()


def build_info() -> str:
    return lib().relm_mp_build_info().decode()


def check(rc: int) -> None:
    if rc == OK:
        return
    msg = last_error()
    if rc == ERR_UNSUPPORTED_MODE:
        raise ValueError(msg)
    raise RuntimeError(msg)


def _dtype(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return F32
    if t.dtype == torch.float64:
        return F64
    raise TypeError(f"relm_mp C ABI supports float32 / float64, got {t.dtype}")


def _ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    assert t.is_contiguous(), "C ABI tensors must be contiguous"
    return t.data_ptr()


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _bytes(n: int, like: torch.Tensor) -> torch.Tensor:
    return torch.empty(max(int(n), 1), dtype=torch.uint8, device=like.device)


def _check_index(t: torch.Tensor) -> None:
    assert t.dtype == torch.int64 and t.dim() == 1 and t.is_contiguous()


# ---- op-level entry points ----------------------------------------------------


def fanout_scatter(x_cat: torch.Tensor, src: torch.Tensor, dst: torch.Tensor, out_rows: int) -> torch.Tensor:
    _check_index(src)
    _check_index(dst)
    emb = x_cat.size(1)
    out = torch.empty(out_rows, emb, dtype=x_cat.dtype, device=x_cat.device)
    ws_n = lib().relm_mp_fanout_scatter_workspace_size(src.numel(), out_rows)
    ws = _bytes(ws_n, x_cat)
    check(
        lib().relm_mp_fanout_scatter(
            _dtype(x_cat), _ptr(x_cat), x_cat.size(0), emb, _ptr(src), _ptr(dst), src.numel(),
            out_rows, _ptr(out), _ptr(ws), ws.numel(), _stream(x_cat),
        )
    )
    return out


def fanout_scatter_backward(grad_out: torch.Tensor, src: torch.Tensor, dst: torch.Tensor, x_rows: int) -> torch.Tensor:
    _check_index(src)
    _check_index(dst)
    emb = grad_out.size(1)
    grad_x = torch.empty(x_rows, emb, dtype=grad_out.dtype, device=grad_out.device)
    ws_n = lib().relm_mp_fanout_scatter_backward_workspace_size(src.numel(), x_rows, emb, _dtype(grad_out))
    ws = _bytes(ws_n, grad_out)
    check(
        lib().relm_mp_fanout_scatter_backward(
            _dtype(grad_out), _ptr(grad_out), grad_out.size(0), emb, _ptr(src), _ptr(dst),
            src.numel(), x_rows, _ptr(grad_x), _ptr(ws), ws.numel(), _stream(grad_out),
        )
    )
    return grad_x


def fanin_reduce(rel_flat: torch.Tensor, flat_src: torch.Tensor, dst_idx: torch.Tensor, dim_size: int, mode: int) -> torch.Tensor:
    _check_index(flat_src)
    _check_index(dst_idx)
    emb = rel_flat.size(1)
    out = torch.empty(dim_size, emb, dtype=rel_flat.dtype, device=rel_flat.device)
    ws_n = lib().relm_mp_fanin_reduce_workspace_size(flat_src.numel(), dim_size, emb, _dtype(rel_flat))
    ws = _bytes(ws_n, rel_flat)
    check(
        lib().relm_mp_fanin_reduce(
            _dtype(rel_flat), _ptr(rel_flat), rel_flat.size(0), emb, _ptr(flat_src), _ptr(dst_idx),
            flat_src.numel(), dim_size, mode, _ptr(out), _ptr(ws), ws.numel(), _stream(rel_flat),
        )
    )
    return out


def fanin_reduce_noalloc(rel_flat: torch.Tensor, flat_src: torch.Tensor, dst_idx: torch.Tensor, dim_size: int,
                        mode: int) -> torch.Tensor:
    """``relm_mp_fanin_reduce_noalloc``: the same op on the library's own device
    scratch (the caller passes inputs and the output only)."""

    _check_index(flat_src)
    _check_index(dst_idx)
    emb = rel_flat.size(1)
    out = torch.empty(dim_size, emb, dtype=rel_flat.dtype, device=rel_flat.device)
    check(
        lib().relm_mp_fanin_reduce_noalloc(
            _dtype(rel_flat), _ptr(rel_flat), rel_flat.size(0), emb, _ptr(flat_src), _ptr(dst_idx),
            flat_src.numel(), dim_size, mode, _ptr(out), _stream(rel_flat),
        )
    )
    return out


NOALLOC_SCRATCH_BYTES = 64 << 20  # RELM_MP_NOALLOC_SCRATCH_BYTES


def fanin_reduce_sum_backward(grad_out: torch.Tensor, flat_src: torch.Tensor, dst_idx: torch.Tensor, rel_rows: int) -> torch.Tensor:
    _check_index(flat_src)
    _check_index(dst_idx)
    emb = grad_out.size(1)
    grad_rel = torch.empty(rel_rows, emb, dtype=grad_out.dtype, device=grad_out.device)
    ws_n = lib().relm_mp_fanin_reduce_sum_backward_workspace_size(flat_src.numel(), rel_rows, emb, _dtype(grad_out))
    ws = _bytes(ws_n, grad_out)
    check(
        lib().relm_mp_fanin_reduce_sum_backward(
            _dtype(grad_out), _ptr(grad_out), grad_out.size(0), emb, _ptr(flat_src), _ptr(dst_idx),
            flat_src.numel(), rel_rows, _ptr(grad_rel), _ptr(ws), ws.numel(), _stream(grad_out),
        )
    )
    return grad_rel


def fanin_reduce_logsumexp_backward(
    grad_out: torch.Tensor,
    rel_flat: torch.Tensor,
    flat_src: torch.Tensor,
    dst_idx: torch.Tensor,
    out: torch.Tensor,
    rel_rows: int,
) -> torch.Tensor:
    _check_index(flat_src)
    _check_index(dst_idx)
    emb = grad_out.size(1)
    grad_rel = torch.empty(rel_rows, emb, dtype=rel_flat.dtype, device=rel_flat.device)
    ws_n = lib().relm_mp_fanin_reduce_logsumexp_backward_workspace_size(
        flat_src.numel(), rel_rows, emb, _dtype(rel_flat)
    )
    ws = _bytes(ws_n, rel_flat)
    check(
        lib().relm_mp_fanin_reduce_logsumexp_backward(
            _dtype(rel_flat), _ptr(grad_out), grad_out.size(0), emb, _ptr(rel_flat), rel_flat.size(0),
            _ptr(flat_src), _ptr(dst_idx), flat_src.numel(), _ptr(out), rel_rows, _ptr(grad_rel),
            _ptr(ws), ws.numel(), _stream(rel_flat),
        )
    )
    return grad_rel


# ---- plans -------------------------------------------------------------------------


class BuiltPlan:
    """A plan descriptor together with the device memory it points into."""

    def __init__(self, plan: Plan, mem: torch.Tensor):
        self.plan = plan
        self.mem = mem

    def _i32(self, ptr: int, n: int) -> torch.Tensor:
        """View of ``n`` int32 values of the plan memory starting at ``ptr``."""

        base = self.mem.data_ptr()
        off = int(ptr) - base
        assert 0 <= off and off + 4 * n <= self.mem.numel(), "pointer outside plan memory"
        return self.mem[off : off + 4 * n].view(torch.int32)

    @property
    def inv(self) -> torch.Tensor:
        if not self.plan.inv:  # identity plan: key k <-> edge k
            k = torch.arange(self.plan.num_keys, dtype=torch.int32, device=self.mem.device)
            return torch.where(k < self.plan.num_edges, k, torch.full_like(k, -1))
        return self._i32(self.plan.inv, self.plan.num_keys)

    @property
    def offsets(self) -> torch.Tensor:
        return self._i32(self.plan.offsets, self.plan.num_keys + 1)

    @property
    def gather_sorted(self) -> torch.Tensor:
        return self._i32(self.plan.gather_sorted, self.plan.num_edges)

    @property
    def keys_sorted(self) -> torch.Tensor:
        """The key of each position of ``gather_sorted``, expanded from the
        offsets (plans keep no sorted keys)."""
        off = self.offsets
        keys = torch.arange(self.plan.num_keys, dtype=torch.int32, device=off.device)
        return torch.repeat_interleave(keys, (off[1:] - off[:-1]).to(torch.int64))

    @property
    def item_first(self) -> torch.Tensor:
        return self._i32(self.plan.item_first, self.plan.num_items + 1)

    @property
    def item_short(self) -> torch.Tensor:
        return self._i32(self.plan.item_short, self.plan.num_items + 1)

    @property
    def short_off(self) -> torch.Tensor:
        return self._i32(self.plan.short_off, self.plan.num_keys + 1)

    @property
    def short_gather(self) -> torch.Tensor:
        return self._i32(self.plan.short_gather, self.plan.num_short)


def inv_plan(keys: torch.Tensor, key_bound: int, gathers: torch.Tensor | None, gather_bound: int,
             key_name: str = "key", gather_name: str = "gather", gather_first: bool = False,
             wait: bool = True, snapshot: bool = False) -> BuiltPlan:
    """Inverse plan; with wait=False the validation stays pending until validate();
    with snapshot=True the plan keeps a snapshot of its indices (plan_match)."""

    _check_index(keys)
    flags = PLAN_SNAPSHOT if snapshot else 0
    mem = _bytes(lib().relm_mp_inv_plan_bytes(key_bound, keys.numel(), flags), keys)
    plan = Plan()
    build = lib().relm_mp_inv_plan_build if wait else lib().relm_mp_inv_plan_build_async
    # the names must outlive a pending validation: keep them on the plan
    names = (key_name.encode(), gather_name.encode())
    check(
        build(
            _ptr(keys), key_bound, names[0], _ptr(gathers), gather_bound,
            names[1], int(gather_first), keys.numel(), flags, _ptr(mem), mem.numel(),
            ctypes.byref(plan), _stream(keys),
        )
    )
    bp = BuiltPlan(plan, mem)
    bp.names = names
    return bp


def validate(bp: BuiltPlan) -> None:
    check(lib().relm_mp_plan_validate(ctypes.byref(bp.plan)))


def csr_plan(keys: torch.Tensor, key_bound: int, gathers: torch.Tensor | None, gather_bound: int,
             key_name: str = "key", gather_name: str = "gather", gather_first: bool = False,
             wait_counts: bool = True) -> BuiltPlan:
    """CSR plan; with wait_counts=False the build returns after validation and the
    host-side statistics stay -1 until read_counts()."""

    _check_index(keys)
    n = keys.numel()
    mem = _bytes(lib().relm_mp_csr_plan_bytes(key_bound, n), keys)
    scratch = _bytes(lib().relm_mp_csr_plan_scratch_bytes(key_bound, n), keys)
    plan = Plan()
    build = lib().relm_mp_csr_plan_build if wait_counts else lib().relm_mp_csr_plan_build_async
    check(
        build(
            _ptr(keys), key_bound, key_name.encode(), _ptr(gathers), gather_bound,
            gather_name.encode(), int(gather_first), n, _ptr(mem), mem.numel(), _ptr(scratch),
            scratch.numel(), ctypes.byref(plan), _stream(keys),
        )
    )
    bp = BuiltPlan(plan, mem)
    bp.scratch = scratch  # the queued build kernels still use it
    return bp


def read_counts(bp: BuiltPlan, like: torch.Tensor) -> None:
    check(lib().relm_mp_plan_read_counts(ctypes.byref(bp.plan), _stream(like)))


def plan_segment_reduce(bp: BuiltPlan, table: torch.Tensor, mode: int, gathers: torch.Tensor | None = None) -> torch.Tensor:
    emb = table.size(1)
    out = torch.empty(bp.plan.num_keys, emb, dtype=table.dtype, device=table.device)
    n = lib().relm_mp_plan_compute_scratch_bytes(ctypes.byref(bp.plan), emb, _dtype(table), mode)
    scratch = _bytes(n, table)
    check(
        lib().relm_mp_plan_segment_reduce(
            _dtype(table), ctypes.byref(bp.plan), _ptr(gathers), _ptr(table), emb, mode, _ptr(out),
            _ptr(scratch), scratch.numel(), _stream(table),
        )
    )
    return out


def plan_segment_sum_scaled(bp: BuiltPlan, table: torch.Tensor, div_kind: int = 0,
                            div_values: torch.Tensor | None = None,
                            base: torch.Tensor | None = None) -> torch.Tensor:
    emb = table.size(1)
    out = torch.empty(bp.plan.num_keys, emb, dtype=table.dtype, device=table.device)
    n = lib().relm_mp_plan_compute_scratch_bytes(ctypes.byref(bp.plan), emb, _dtype(table), 0)
    scratch = _bytes(n, table)
    check(
        lib().relm_mp_plan_segment_sum_scaled(
            _dtype(table), ctypes.byref(bp.plan), _ptr(table), emb, div_kind, _ptr(div_values),
            _ptr(base), _ptr(out), _ptr(scratch), scratch.numel(), _stream(table),
        )
    )
    return out


def plan_segment_sum_msgdiv(bp: BuiltPlan, table: torch.Tensor, div_plan: BuiltPlan,
                            base: torch.Tensor | None = None) -> torch.Tensor:
    """``relm_mp_plan_segment_sum_msgdiv``: each gathered row divided by its count
    in ``div_plan`` (a CSR plan keyed by the table's rows) before it is added."""
    emb = table.size(1)
    out = torch.empty(bp.plan.num_keys, emb, dtype=table.dtype, device=table.device)
    n = lib().relm_mp_plan_compute_scratch_bytes(ctypes.byref(bp.plan), emb, _dtype(table), 0)
    scratch = _bytes(n, table)
    check(
        lib().relm_mp_plan_segment_sum_msgdiv(
            _dtype(table), ctypes.byref(bp.plan), _ptr(table), emb, div_plan.plan.offsets,
            _ptr(base), _ptr(out), _ptr(scratch), scratch.numel(), _stream(table),
        )
    )
    return out


def plan_logsumexp_backward(bp: BuiltPlan, grad_out: torch.Tensor, out: torch.Tensor, rel_flat: torch.Tensor,
                            gathers: torch.Tensor | None = None) -> torch.Tensor:
    emb = grad_out.size(1)
    grad_rel = torch.empty(bp.plan.num_keys, emb, dtype=rel_flat.dtype, device=rel_flat.device)
    n = lib().relm_mp_plan_compute_scratch_bytes(ctypes.byref(bp.plan), emb, _dtype(rel_flat), 0)
    scratch = _bytes(n, rel_flat)
    check(
        lib().relm_mp_plan_logsumexp_backward(
            _dtype(rel_flat), ctypes.byref(bp.plan), _ptr(gathers), _ptr(grad_out), _ptr(out),
            _ptr(rel_flat), emb, _ptr(grad_rel), _ptr(scratch), scratch.numel(), _stream(rel_flat),
        )
    )
    return grad_rel


def plan_fanin_backward_by_dst(bp: BuiltPlan, dst_idx: torch.Tensor, mode: int, grad_out: torch.Tensor,
                               rel_rows: int, out: torch.Tensor | None = None,
                               rel_flat: torch.Tensor | None = None) -> torch.Tensor:
    """Backward of fanin_reduce over the forward's CSR plan (keys = dst_idx,
    gathers = flat_src) when flat_src is the identity."""

    _check_index(dst_idx)
    emb = grad_out.size(1)
    grad_rel = torch.empty(rel_rows, emb, dtype=grad_out.dtype, device=grad_out.device)
    check(
        lib().relm_mp_plan_fanin_backward_by_dst(
            _dtype(grad_out), ctypes.byref(bp.plan), _ptr(dst_idx), mode, _ptr(grad_out), _ptr(out),
            _ptr(rel_flat), emb, _ptr(grad_rel), rel_rows, _stream(grad_out),
        )
    )
    return grad_rel


def plan_fanin_backward_by_src(bp: BuiltPlan, mode: int, grad_out: torch.Tensor, rel_rows: int,
                               out: torch.Tensor | None = None,
                               rel_flat: torch.Tensor | None = None) -> tuple[torch.Tensor, int]:
    """Backward of fanin_reduce over the forward's CSR plan when flat_src is not
    the identity: (grad_rel, collisions); grad_rel is the result when
    collisions == 0."""

    emb = grad_out.size(1)
    grad_rel = torch.empty(rel_rows, emb, dtype=grad_out.dtype, device=grad_out.device)
    mem = _bytes(lib().relm_mp_inv_plan_bytes(rel_rows, bp.plan.num_edges, 0), grad_out)
    collisions = ctypes.c_int64(-1)
    check(
        lib().relm_mp_plan_fanin_backward_by_src(
            _dtype(grad_out), ctypes.byref(bp.plan), mode, _ptr(grad_out), _ptr(out), _ptr(rel_flat), emb,
            _ptr(grad_rel), rel_rows, _ptr(mem), mem.numel(), 0, ctypes.byref(collisions), _stream(grad_out),
        )
    )
    return grad_rel, collisions.value


def identity_inv_plan(num_keys: int, num_edges: int, num_gather: int) -> BuiltPlan:
    """Inverse plan that maps key k to edge k (k < num_edges): ``inv`` is NULL."""

    plan = Plan()
    plan.kind = PLAN_INVERSE
    plan.num_keys, plan.num_edges, plan.num_gather = num_keys, num_edges, num_gather
    return BuiltPlan(plan, torch.empty(0, dtype=torch.uint8))


def plan_gather_last(bp: BuiltPlan, table: torch.Tensor, gathers: torch.Tensor | None = None) -> torch.Tensor:
    emb = table.size(1)
    out = torch.empty(bp.plan.num_keys, emb, dtype=table.dtype, device=table.device)
    check(
        lib().relm_mp_plan_gather_last(
            _dtype(table), ctypes.byref(bp.plan), _ptr(gathers), _ptr(table), emb, _ptr(out),
            _stream(table),
        )
    )
    return out


def _slot_base(mat: torch.Tensor, col_offset: int) -> int:
    assert mat.dim() == 2 and mat.stride(1) == 1
    return mat.data_ptr() + col_offset * mat.element_size()


def plan_gather_last_grouped(bp: BuiltPlan, table: torch.Tensor, out: torch.Tensor, col_offset: int,
                             group: int, gathers: torch.Tensor | None = None) -> torch.Tensor:
    """Gather of the plan's rows into ``out`` [lines, width]: row k goes to line
    k // group, columns col_offset + (k % group) * D ... + D."""

    emb = table.size(1)
    check(
        lib().relm_mp_plan_gather_last_grouped(
            _dtype(table), ctypes.byref(bp.plan), _ptr(gathers), _ptr(table), emb, group,
            out.stride(0), _slot_base(out, col_offset), _stream(table),
        )
    )
    return out


def plan_segment_sum_grouped(bp: BuiltPlan, table: torch.Tensor, col_offset: int, group: int,
                             emb: int) -> torch.Tensor:
    """Segment sums over a CSR plan whose gathered rows are read from the
    argument columns of ``table`` [lines, width] (row r = line r // group,
    columns col_offset + (r % group) * emb ... + emb)."""

    out = torch.empty(bp.plan.num_keys, emb, dtype=table.dtype, device=table.device)
    n = lib().relm_mp_plan_compute_scratch_bytes(ctypes.byref(bp.plan), emb, _dtype(table), 0)
    scratch = _bytes(n, table)
    check(
        lib().relm_mp_plan_segment_sum_grouped(
            _dtype(table), ctypes.byref(bp.plan), _slot_base(table, col_offset),
            table.size(0) * group, emb, group, table.stride(0), _ptr(out), _ptr(scratch),
            scratch.numel(), _stream(table),
        )
    )
    return out


__all__ = [name for name in dir() if not name.startswith("_")]


def pack_index(parts: list[tuple], write_b: bool = True) -> tuple[torch.Tensor, torch.Tensor | None]:
    """``relm_mp_pack_index`` over parts ``(a, b, a_mul, a_add, b_mul, b_add)``
    (contiguous int64 device tensors of equal length); returns (out_a, out_b)."""

    if not parts:
        raise ValueError("pack_index needs at least one part")
    like = parts[0][0]
    descs = (IndexPart * len(parts))()
    total = 0
    for d, (a, b, a_mul, a_add, b_mul, b_add) in zip(descs, parts):
        _check_index(a)
        _check_index(b)
        if a.numel() != b.numel():
            raise ValueError("index parts of unequal length")
        d.a, d.b, d.n = _ptr(a), _ptr(b), a.numel()
        d.a_mul, d.a_add, d.b_mul, d.b_add = int(a_mul), int(a_add), int(b_mul), int(b_add)
        total += a.numel()
    out_a = torch.empty(total, dtype=torch.int64, device=like.device)
    out_b = torch.empty(total, dtype=torch.int64, device=like.device) if write_b else None
    check(lib().relm_mp_pack_index(descs, len(parts), _ptr(out_a), _ptr(out_b), _stream(like)))
    return out_a, out_b


def _starts(range_start: list[int]):
    arr = (ctypes.c_int64 * len(range_start))(*range_start)
    return arr, len(range_start) - 1


def film_mish(s: torch.Tensor, range_start: list[int], gamma: torch.Tensor, beta: torch.Tensor,
              add: torch.Tensor | None = None) -> torch.Tensor:
    """``relm_mp_film_mish`` on contiguous float32 device tensors."""

    y = torch.empty_like(s)
    starts, k = _starts(range_start)
    check(lib().relm_mp_film_mish(_ptr(s), s.size(0), s.size(1), starts, k, _ptr(gamma), _ptr(beta),
                                  _ptr(add) if add is not None else None, _ptr(y), _stream(s)))
    return y


def film_mish_backward(dy: torch.Tensor, s: torch.Tensor, range_start: list[int], gamma: torch.Tensor,
                       beta: torch.Tensor, add: torch.Tensor | None = None):
    """``relm_mp_film_mish_backward``: (ds, per-block partial sums [blocks, 2, width], float64)."""

    starts, k = _starts(range_start)
    blocks = lib().relm_mp_film_mish_blocks(starts, k)
    ds = torch.empty_like(s)
    partial = torch.empty(max(blocks, 1), 2, s.size(1), dtype=torch.float64, device=s.device)
    check(lib().relm_mp_film_mish_backward(_ptr(s), _ptr(dy), s.size(0), s.size(1), starts, k,
                                           _ptr(gamma), _ptr(beta), _ptr(add) if add is not None else None,
                                           _ptr(ds), _ptr(partial), blocks, _stream(s)))
    return ds, partial[:blocks]


def plan_match(keys: torch.Tensor, gathers: torch.Tensor | None, plans: list[BuiltPlan]) -> list[bool]:
    """``relm_mp_plan_match``: which plans were built from indices equal to (keys, gathers)."""

    _check_index(keys)
    if gathers is not None:
        _check_index(gathers)
    k = len(plans)
    arr = (_PP * max(k, 1))(*[ctypes.pointer(bp.plan) for bp in plans])
    match = (ctypes.c_int32 * max(k, 1))()
    ws = _bytes(lib().relm_mp_plan_match_workspace_size(), keys)
    check(lib().relm_mp_plan_match(_ptr(keys), _ptr(gathers), keys.numel(), arr, k, match,
                                   _ptr(ws), ws.numel(), _stream(keys)))
    return [bool(match[i]) for i in range(k)]


DIV_NONE, DIV_SEGMENT, DIV_VALUES = 0, 1, 2


def rows_scale(inp: torch.Tensor | None, rows: int, emb: int, like: torch.Tensor, *,
               gather: torch.Tensor | None = None, div_kind: int = DIV_NONE,
               div_offsets: torch.Tensor | None = None, div_values: torch.Tensor | None = None,
               base: torch.Tensor | None = None) -> torch.Tensor:
    """``relm_mp_rows_scale`` into a new [rows, emb] tensor of like's dtype."""

    out = torch.empty(rows, emb, dtype=like.dtype, device=like.device)
    check(lib().relm_mp_rows_scale(_dtype(like), _ptr(inp), _ptr(gather), div_kind, _ptr(div_offsets),
                                   _ptr(div_values), _ptr(base), rows, emb, _ptr(out), _stream(like)))
    return out
