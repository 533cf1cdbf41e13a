"""Tensor-level entry points of the gfx950 kernels: every function takes and returns torch tensors on the GPU and
enqueues HIP kernels on torch's current stream (no host synchronisation unless a result is read back). These
are what the reference-compatible modules (codes, frame, nested, quantize, compiler, artifact) are built on."""

from __future__ import annotations

import contextlib
import ctypes
from functools import lru_cache

import numpy as np
import torch

from . import _abi
from ._abi import check, ld, lib, need, ptr, stream, workspace
from .hadamard import hadamard_factors, rht_signs


class LinAlgError(torch.linalg.LinAlgError if hasattr(torch.linalg, "LinAlgError") else RuntimeError):
    pass


# ----------------------------------------------------------------------------- Viterbi (codes.py:151-181)


BIG_L = 13  # tables of 2^13 states and more go to the 1024-thread kernels (fp16-exact tables)
MERGED_SMALL_L = 12  # below BIG_L, the state width whose row groups go through one launch per lazy block


def half_bits(C: torch.Tensor) -> torch.Tensor:
    """The fp16 bit patterns (int16 tensor) of a table whose values fp16 represents exactly; raises otherwise."""
    c32 = C.to(torch.float32)
    h = c32.to(torch.float16)
    if not torch.equal(h.to(torch.float32), c32):
        raise NotImplementedError("the 2^13..2^16-state kernels take tables whose values are exact in fp16")
    return h.view(torch.int16).contiguous()


def search16(L: int, k: int, C: torch.Tensor) -> bool:
    """Whether the standalone search at (L, k) goes to the 2^13..2^16-state kernels (lamq_viterbi16_rows: k <= L - 12
    and k <= 4, a table exact in fp16); otherwise lamq_viterbi_rows takes it (L <= 12 with k <= 4 on the kernels built
    per (L, k); k = 5..8, or up to 2^14 states with any float32 table, on its wide search)."""
    if L < BIG_L or k > min(4, L - 12):
        return False
    c32 = C.to(torch.float32)
    return bool(torch.equal(c32.to(torch.float16).to(torch.float32), c32))


def viterbi_rows(x: torch.Tensor, C: torch.Tensor, L: int, k: int, start: torch.Tensor | None = None,
                 C16: torch.Tensor | None = None) -> torch.Tensor:
    """x [B, T] float32, C [2^L] float32, start None or [B] int32 -> states [B, T] int32. C16: C's fp16 bit patterns,
    given when the caller has them (the 2^13..2^16-state kernels read those)."""
    need(x, torch.float32, "x", 2)
    need(C, torch.float32, "C", 1)
    if C.numel() != 1 << L:
        raise ValueError("the table must have 2^L entries")
    B, T = x.shape
    out = torch.empty(B, T, dtype=torch.int32, device=x.device)
    st = None
    if start is not None:
        st = start.to(device=x.device, dtype=torch.int32).contiguous()
        if st.numel() != B:
            raise ValueError("one start state per row")
    if C16 is not None or search16(L, k, C):
        h = half_bits(C) if C16 is None else C16
        nbytes = lib().lamq_viterbi16_workspace_size(B, T, L, k)
        ws = workspace(nbytes, x.device)
        check(lib().lamq_viterbi16_rows(ptr(x), B, T, ld(x), ptr(h), L, k, ptr(st), ptr(out), T, ptr(ws), nbytes,
                                        stream(x.device)), "viterbi16")
        return out
    nbytes = lib().lamq_viterbi_workspace_size(B, T, L, k)
    ws = workspace(nbytes, x.device)
    check(lib().lamq_viterbi_rows(ptr(x), B, T, ld(x), ptr(C), L, k, ptr(st), ptr(out), T, ptr(ws), nbytes,
                                  stream(x.device)), "viterbi")
    return out


# ----------------------------------------------------------------------------- randomized Hadamard transforms


_UPLOADS: dict = {}  # key -> (device tensors, event after their copy), oldest first
_UPLOADS_MAX = 512


def _uploaded(key, make, dev: str) -> tuple:
    """Small host-made tables (int8 signs and Hadamard factors) on the device, cached by key: the first use copies
    them from pinned memory without making the host wait (a blocking copy would wait for the current stream and,
    through it, for every stream it waits on); every use makes the current stream wait for that copy (an event, no
    host wait) and marks the tensors as used by it, so an evicted entry's memory is not reused while a kernel on
    that stream may still read it."""
    cur = torch.cuda.current_stream(torch.device(dev))
    hit = _UPLOADS.get(key)
    if hit is None:
        ts = tuple(t.to(dev, non_blocking=True) for t in (x.to(torch.int8).contiguous().pin_memory() for x in make()))
        ev = torch.cuda.Event()
        ev.record(cur)
        hit = (ts, ev)
        while len(_UPLOADS) >= _UPLOADS_MAX:
            _UPLOADS.pop(next(iter(_UPLOADS)))
        _UPLOADS[key] = hit
    else:
        cur.wait_event(hit[1])
        for t in hit[0]:
            t.record_stream(cur)
    return hit[0]


def _factors(n: int, dev: str):
    return _uploaded(("factors", n, dev), lambda: hadamard_factors(n), dev)


def _signs(n: int, seed: int, dev: str):
    return _uploaded(("signs", n, seed, dev), lambda: (rht_signs(n, seed),), dev)[0]


def rht_rows(X: torch.Tensor, seed: int, inverse: bool = False, want_rms: bool = False, out: torch.Tensor | None = None):
    """X @ R^T (or X @ R with inverse) for R = rht(n, seed), row by row in Kronecker-factored form; optionally the
    row RMS max(sqrt(mean x^2), 1e-12) of the result (codes.py:436)."""
    need(X, torch.float64, "X", 2)
    rows, n = X.shape
    dev = str(X.device)
    A, B = _factors(n, dev)
    s = _signs(n, seed, dev)
    y = torch.empty_like(X, memory_format=torch.contiguous_format) if out is None else out
    rms = torch.empty(rows, dtype=torch.float64, device=X.device) if want_rms else None
    check(lib().lamq_rht_rows(ptr(X), rows, n, ld(X), ptr(y), ld(y), ptr(s), ptr(A), A.shape[0], ptr(B), B.shape[0],
                              1 if inverse else 0, ptr(rms), stream(X.device)), "rht_rows")
    return (y, rms) if want_rms else y


def device_rows(groups: list, dev) -> list:
    """Each row group's row indices ({"rows": [...]}) as an int64 tensor on the device, through one pinned buffer
    and one asynchronous copy: no per-group upload that would make the host wait for the stream."""
    sizes = [len(g["rows"]) for g in groups]
    host = torch.empty(sum(sizes), dtype=torch.int64, pin_memory=True)
    if sizes and sum(sizes):
        host.numpy()[:] = np.concatenate([np.asarray(g["rows"], dtype=np.int64).reshape(-1) for g in groups])
    return list(torch.split(host.to(dev, non_blocking=True), sizes))


def rht_flops(rows: int, n: int) -> float:
    """Algorithmic fp64 work of rht_rows over `rows` rows of width n: the two Kronecker factors' products, 2n(a + b)
    flops a row (a x b = n)."""
    a, b = _factor_sizes(n)
    return 2.0 * rows * n * (a + b)


@lru_cache(maxsize=64)
def _factor_sizes(n: int) -> tuple:
    A, B = hadamard_factors(n)
    return A.shape[0], B.shape[0]


def row_rms(X: torch.Tensor) -> torch.Tensor:
    """S_r = max(sqrt(mean_j X_rj^2), 1e-12) (codes.py:436)."""
    need(X, torch.float64, "X", 2)
    S = torch.empty(X.shape[0], dtype=torch.float64, device=X.device)
    check(lib().lamq_row_rms(ptr(X), X.shape[0], X.shape[1], ld(X), ptr(S), stream(X.device)), "row_rms")
    return S


def transpose(X: torch.Tensor) -> torch.Tensor:
    need(X, torch.float64, "X", 2)
    r, c = X.shape
    out = torch.empty(c, r, dtype=torch.float64, device=X.device)
    check(lib().lamq_transpose_f64(ptr(X), r, c, ld(X), ptr(out), r, stream(X.device)), "transpose")
    return out


def rotate_hessian(H: torch.Tensor, seed: int) -> torch.Tensor:
    """R H R^T for R = rht(n, seed) (codes.py:439): the rows of H, a transpose, the rows again."""
    Y = rht_rows(H, seed)
    return rht_rows(transpose(Y), seed)


def rotate_columns(X: torch.Tensor, seed: int) -> torch.Tensor:
    """R X for R = rht(rows, seed): the output-side rotation of incoherence (codes.py:253-263)."""
    return transpose(rht_rows(transpose(X), seed))


def unrotate_columns(X: torch.Tensor, seed: int) -> torch.Tensor:
    """R^T X."""
    return transpose(rht_rows(transpose(X), seed, inverse=True))


# ----------------------------------------------------------------------------- environment (frame.py:515-522)


CHOL_KEEP_DEAD = 1


_SIDE_STREAMS: dict = {}


def _side_stream(dev: torch.device) -> torch.cuda.Stream:
    """The stream on which the factor's inverse half runs beside the current stream: one per (device, calling stream),
    made on first use at the default priority, so that factorizations enqueued on different streams stay independent
    (lamq_chol_inv_upper_ex forks from and joins back into the calling stream)."""
    cur = torch.cuda.current_stream(dev)
    key = (cur.device.index, cur.cuda_stream)
    if key not in _SIDE_STREAMS:
        _SIDE_STREAMS[key] = torch.cuda.Stream(device=cur.device)
    return _SIDE_STREAMS[key]


def chol_inv_upper(H: torch.Tensor, damp: float = 0.01, raise_on_fail: bool = True, keep_dead: bool = False):
    """(Hd, U, dead, info): the damped H, the upper Cholesky factor of its inverse, the dead-column mask and the
    failing pivot (0 when H is positive definite after damping; raises LinAlgError then unless told not to).
    keep_dead: zero diagonal entries stay zero (ldlq_factor's damping) instead of becoming 1 (Environment's)."""
    need(H, torch.float64, "H", 2)
    n = H.shape[0]
    if H.shape[1] != n:
        raise ValueError("H must be square")
    Hd = torch.empty(n, n, dtype=torch.float64, device=H.device)
    U = torch.empty(n, n, dtype=torch.float64, device=H.device)
    dead = torch.empty(n, dtype=torch.uint8, device=H.device)
    info = torch.empty(1, dtype=torch.int32, device=H.device)
    nbytes = lib().lamq_chol_inv_upper_workspace_size(n)
    ws = workspace(nbytes, H.device)
    check(lib().lamq_chol_inv_upper_ex(ptr(H), n, ld(H), float(damp), CHOL_KEEP_DEAD if keep_dead else 0, ptr(Hd), n,
                                       ptr(U), n, ptr(dead), ptr(info), ptr(ws), nbytes, stream(H.device),
                                       _side_stream(H.device).cuda_stream), "chol_inv_upper")
    if raise_on_fail:
        bad = int(info.item())
        if bad:
            raise LinAlgError(f"linalg.cholesky: the leading minor of order {bad} is not positive-definite")
    return Hd, U, dead.bool(), info


# ----------------------------------------------------------------------------- the sweeps (syntax.py:86-124)


FUSED_WMAX, FUSED_TV = 16, 24  # the fused block kernels' widest block and longest search (width + look)


def fused_trellis(L: int, k: int, width: int, look: int, table64: torch.Tensor) -> bool:
    """Whether the fused row-trellis block kernels take (L, k, width, look) with this table: L <= 12 with k <=
    min(4, L - 1), or 13 <= L <= 16 with k <= min(4, L - 12) and a table exact in fp16; width <= 16 and width + look
    <= 24. Other row trellises go through the generic sweep with the standalone search (codes.ldlq_words)."""
    if not (1 <= width <= FUSED_WMAX and look >= 0 and width + look <= FUSED_TV):
        return False
    if L <= 12:
        return 1 <= k <= min(4, L - 1)
    return search16(L, k, table64) and L <= 16


def ldlq_trellis(X: torch.Tensor, S: torch.Tensor, U: torch.Tensor, table64: torch.Tensor, L: int, k: int,
                 width: int = 16, look: int = 8, lazy: int = 128, dead: torch.Tensor | None = None,
                 table32: torch.Tensor | None = None, events: dict | None = None) -> torch.Tensor:
    """States [m, n] int32 of the row-trellis block LDLQ of X (rotated rows, not divided by S) under U.
    events: optional dict; each launch of the block kernel and of the trailing update is bracketed by a pair of
    torch.cuda.Event on this stream, appended to events["block"] and events["trailing"]."""
    return ldlq_trellis_groups(X, S, U, [(X.shape[0], k, table64, table32)], L, width, look, lazy, dead, events)


def ldlq_trellis_groups(X: torch.Tensor, S: torch.Tensor, U: torch.Tensor, groups: list, L: int, width: int = 16,
                        look: int = 8, lazy: int = 128, dead: torch.Tensor | None = None,
                        events: dict | None = None, concurrent: bool | None = None) -> torch.Tensor:
    """ldlq_trellis over consecutive row groups that share U but not the code: groups = [(rows, k, table64,
    table32 or None)] in row order, summing to X's rows. Rows do not interact (the block kernel and the trailing
    update work row by row), so each group's sweep is independent of the others. With 16-bit states (L >= BIG_L) and
    at L = 12 (MERGED_SMALL_L) all groups go through one launch per lazy block (lamq_ldlq_trellis16_block_groups,
    lamq_ldlq_trellis_block_groups) and one trailing product over all rows. At other L, with `concurrent` (the
    default without events) every group runs its whole sweep, block kernels and its own trailing updates, on a stream
    of its own. Either way the results are those of sweeping the groups one after the other. With events every
    launch is timed on the caller's stream in turn."""
    check_tables(groups, L)
    need(X, torch.float64, "X", 2)
    need(U, torch.float64, "U", 2)
    need(S, torch.float64, "S", 1)
    m, n = X.shape
    if sum(int(g[0]) for g in groups) != m:
        raise ValueError("the row groups must cover X's rows")
    if lazy % width:
        raise ValueError("lazy must be a multiple of width and of block")
    T = X.clone(memory_format=torch.contiguous_format)
    dev = X.device
    if dead is not None:
        dd = dead.to(device=dev, dtype=torch.uint8).contiguous()
        check(lib().lamq_zero_columns(ptr(T), m, n, n, ptr(dd), stream(dev)), "zero_columns")
    parts = []
    r0 = 0
    for rows, k, table64, table32 in groups:
        need(table64, torch.float64, "table64", 1)
        if L >= BIG_L:
            t32 = half_bits(table64) if table32 is None or table32.dtype != torch.int16 else table32
        else:
            t32 = table64.to(torch.float32) if table32 is None else table32
        if rows:
            parts.append((r0, int(rows), int(k), table64, t32))
        r0 += int(rows)
    # the 16-bit-state block kernels: a group whose search keeps its back-pointers outside LDS (2^15 groups) gets a
    # workspace of its own, allocated here on the caller's stream before the fork
    ws = {}
    if L >= BIG_L:
        for r0, rows, k, _, _ in parts:
            nb = lib().lamq_ldlq_trellis16_block_workspace_size(rows, L, k)
            if nb:
                ws[r0] = torch.empty(nb, dtype=torch.uint8, device=dev)

    def block(Tp, rows, r0, k, table64, t32, b0, b1, zb, pre, st_):
        args = (ptr(Tp), rows, n, n, ptr(U), ld(U), vp(S.data_ptr() + 8 * r0), ptr(table64), ptr(t32), L, k, b0, b1, width,
                look, vp(state.data_ptr() + 4 * r0), vp(states.data_ptr() + 4 * r0 * n), n, ptr(zb), outer, pre)
        if L < BIG_L:
            return lib().lamq_ldlq_trellis_block(*args, st_)
        w = ws.get(r0)
        if w is None:
            return lib().lamq_ldlq_trellis16_block(*args, st_)
        return lib().lamq_ldlq_trellis16_block_ws(*args, ptr(w), w.numel(), st_)
    state = torch.zeros(m, dtype=torch.int32, device=dev)
    states = torch.empty(m, n, dtype=torch.int32, device=dev)
    outer = _outer_run(lazy)
    Z = torch.empty(m, outer, dtype=torch.float64, device=dev)
    # the 16-bit-state groups go through one launch per lazy block (lamq_ldlq_trellis16_block_groups): every group's
    # rows in one grid, so no group's launch ends in a tail of idle CUs and no stream per group is needed
    merged = None
    if (L >= BIG_L or L == MERGED_SMALL_L) and len(parts) > 1:
        # the grid takes the groups in the table's order, widest first: the costliest rows are dispatched first, so
        # the launch ends on its cheapest rows (a shorter tail of partly idle CUs); rows are independent, so the
        # order changes no result
        order = sorted(parts, key=lambda p: -p[2])
        if L >= BIG_L:
            merged = (_abi.TrellisGroup * len(parts))()
            for i, (r0, rows, k, table64, t32) in enumerate(order):
                w = ws.get(r0)
                merged[i] = _abi.TrellisGroup(r0, rows, k, table64.data_ptr(), t32.data_ptr(),
                                              None if w is None else w.data_ptr(), 0 if w is None else w.numel())
        else:
            merged = (_abi.TrellisGroup32 * len(parts))()
            for i, (r0, rows, k, table64, t32) in enumerate(order):
                merged[i] = _abi.TrellisGroup32(r0, rows, k, table64.data_ptr(), t32.data_ptr())
    if concurrent is None:
        concurrent = events is None
    main = torch.cuda.current_stream(dev)
    lanes = _group_streams(dev) if concurrent and len(parts) > 1 and merged is None else [main]
    for ln in lanes:
        if ln is not main:
            ln.wait_stream(main)
    vp = ctypes.c_void_p
    # each group's rows as views: T, Z and the outputs of rows [r0, r0 + rows)
    views = [(T.narrow(0, r0, rows), Z.narrow(0, r0, rows)) for r0, rows, _, _, _ in parts]
    # per block, a narrow product updates the rest of its run (_refit_run); the run's last block reads its look-ahead
    # past the run with the run's earlier blocks applied in the kernel (pre), and one product per run updates every
    # column past the run (_refit_rest)
    for B0 in range(0, n, outer):
        B1 = min(B0 + outer, n)
        for b0 in range(B0, B1, lazy):
            b1 = min(b0 + lazy, n)
            pre = b0 - B0 if b1 == B1 else 0
            if merged is not None:
                ev = _event_pair(events, "block")
                fn = lib().lamq_ldlq_trellis16_block_groups if L >= BIG_L else lib().lamq_ldlq_trellis_block_groups
                check(fn(ptr(T), m, n, n, ptr(U), ld(U), ptr(S), L, ctypes.addressof(merged), len(parts), b0, b1, width,
                         look, ptr(state), ptr(states), n, vp(Z.data_ptr() + 8 * (b0 - B0)), outer, pre, stream(dev)),
                      "ldlq_trellis_block_groups")
                _event_end(ev)
            for p, (r0, rows, k, table64, t32) in enumerate(parts if merged is None else ()):
                Tp, Zp = views[p]
                with torch.cuda.stream(lanes[p % len(lanes)]):
                    zb = Zp[:, b0 - B0 :]
                    ev = _event_pair(events, "block")
                    check(block(Tp, rows, r0, k, table64, t32, b0, b1, zb, pre, stream(dev)), "ldlq_trellis_block")
                    _event_end(ev)
                    if len(lanes) > 1:
                        _refit_run(Tp, U, zb, b0, b1, B1, 0, events)
            if len(lanes) == 1:  # one product over every group's rows
                _refit_run(T, U, Z[:, b0 - B0 :], b0, b1, B1, 0, events)
        if len(lanes) == 1:
            _refit_rest(T, U, Z, B0, B1, 0, events)
        else:
            for p, (Tp, Zp) in enumerate(views):
                with torch.cuda.stream(lanes[p % len(lanes)]):
                    _refit_rest(Tp, U, Zp, B0, B1, 0, events)
    for ln in lanes:
        if ln is not main:
            main.wait_stream(ln)
    return states


def check_tables(groups: list, L: int):
    """Every group's table has exactly 2^L entries: the float64 table, and the float32 (L < 13) or fp16-bit int16
    (L >= 13) copy when one is given. The kernels read 2^L entries of each, so a shorter table would be read past its
    end."""
    if not 1 <= L <= 16:
        raise ValueError("L must lie in 1..16")
    for g in groups:
        t64, t32 = g[2], g[3] if len(g) > 3 else None
        if not isinstance(t64, torch.Tensor) or t64.dim() != 1 or t64.numel() != 1 << L:
            raise ValueError(f"a trellis table must be a 1-d tensor of 2^L = {1 << L} entries")
        if t32 is not None:
            want = torch.int16 if L >= BIG_L else torch.float32
            if t32.dim() != 1 or t32.numel() != 1 << L or (t32.dtype != want and not (L >= BIG_L and
                                                                                       t32.dtype == torch.float32)):
                raise ValueError(f"the search copy of a trellis table must be a 1-d {want} tensor of 2^L = {1 << L} "
                                 "entries")


_GROUP_STREAMS: dict = {}
GROUP_STREAMS = 4  # streams per device for concurrent row groups (the box's hardware queues per process)


def _group_streams(dev: torch.device) -> list:
    """The device's streams for concurrent row groups (default priority), made once per process."""
    key = torch.device(dev).index if torch.device(dev).index is not None else torch.cuda.current_device()
    if key not in _GROUP_STREAMS:
        _GROUP_STREAMS[key] = [torch.cuda.Stream(device=torch.device("cuda", key)) for _ in range(GROUP_STREAMS)]
    return _GROUP_STREAMS[key]


def _outer_run(lazy: int) -> int:
    """Columns whose trailing updates are gathered into one product: a multiple of lazy, 512 at lazy = 128."""
    return lazy * max(1, 512 // lazy)


def _refit_run(T, U, zb, b0, b1, B1, look, events):
    """The trailing update of lazy block [b0, b1) restricted to the columns its outer run still reads: [b1, B1 + look)
    (the run's later blocks and the look-ahead of its last one)."""
    m, n = T.shape
    e1 = min(B1 + look, n)
    if b1 >= e1:
        return
    ev = _event_pair(events, "trailing")
    # T[:, b1:e1] -= Z U[b0:b1, b1:e1]: the entry point on the first e1 columns
    check(lib().lamq_trailing_update_f64(ptr(T), m, e1, ld(T), ptr(zb), ld(zb), ptr(U), ld(U), b0, b1, stream(T.device)),
          "trailing_update")
    _event_end(ev)


def _refit_rest(T, U, Z, B0, B1, look, events):
    """The columns past the outer run [B0, B1), past its first `look` (which the narrow products already updated), get
    the run's blocks at once: T[:, c0:] -= Z[:, :B1-B0] U[B0:B1, c0:] with c0 = B1 + look (syntax.py:123 summed over
    the run's blocks)."""
    m, n = T.shape
    c0 = B1 + look
    if c0 >= n:
        return
    sh = c0 - B1  # shift the column origin so that the entry point's b1 lands on c0
    ev = _event_pair(events, "trailing")
    check(lib().lamq_trailing_update_f64(T.data_ptr() + 8 * sh, m, n - sh, ld(T), ptr(Z), ld(Z), U.data_ptr() + 8 * sh,
                                         ld(U), B0, B1, stream(T.device)), "trailing_update")
    _event_end(ev)


def _event_pair(events: dict | None, key: str):
    if events is None:
        return None
    _lead(events)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    events.setdefault(key, []).append((a, b))
    return b


def _event_end(ev):
    if ev is not None:
        ev.record()


def viterbi_ops_per_row_step(L: int, k: int) -> int:
    """Algorithmic fp32 operations of one trellis step of one row: a subtraction, a square and an addition per state,
    and 2^k - 1 comparisons per group of 2^k predecessors."""
    return 3 * (1 << L) + ((1 << k) - 1) * (1 << (L - k))


def trellis_call_lengths(n: int, width: int = 16, look: int = 8, lazy: int = 128) -> list[list[int]]:
    """Positions of each search call per row, by lazy block of the row-trellis sweep: the w settled columns of the
    call and its look-ahead columns (codes.py:386-404 via syntax.py:106-123)."""
    out = []
    for b0 in range(0, n, lazy):
        b1 = min(b0 + lazy, n)
        calls = []
        for j in range(b0, b1, width):
            w = min(width, b1 - j)
            calls.append(w + min(look, n - j - w))
        out.append(calls)
    return out


def trellis_row_steps(n: int, width: int = 16, look: int = 8, lazy: int = 128) -> list[int]:
    """Trellis positions searched per row in each lazy block of the row-trellis sweep (the settled and the look-ahead
    columns of every call)."""
    return [sum(c) for c in trellis_call_lengths(n, width, look, lazy)]


def viterbi_search_ops(L: int, k: int, T: int) -> int:
    """Algorithmic fp32 operations of one search of T positions from a fixed start state, counting reachable states
    only. Position t reaches the 2^a states, a = min(L, k (t + 1)), whose low a bits are free: each costs a
    subtraction, a square and an addition. Forming position t's costs takes 2^k - 1 comparisons in each group of
    predecessors (the states sharing their low L - k bits) only as far as the group holds several reachable ones:
    with a' = min(L, k t) reachable bits at t - 1, 2^min(a', L - k) groups of 2^max(0, a' - L + k) members. Once
    k t >= L every term equals viterbi_ops_per_row_step(L, k); the shorter first positions are the part of the
    reference's full-array recurrence (codes.py:164-179) whose states are +inf."""
    ops = 0
    for t in range(T):
        a = min(L, k * (t + 1))
        ops += 3 * (1 << a)
        if t > 0:
            ap = min(L, k * t)
            members = 1 << max(0, ap - (L - k))
            ops += (members - 1) * (1 << min(ap, L - k))
    return ops


def trellis_block_ops(n: int, L: int, k: int, width: int = 16, look: int = 8, lazy: int = 128) -> list[int]:
    """Reachable-state operations (viterbi_search_ops) of the searches of one row, by lazy block. Every call of the
    row-trellis sweep has a fixed start state: the previous call's last settled state, 0 for the first."""
    return [sum(viterbi_search_ops(L, k, T) for T in c) for c in trellis_call_lengths(n, width, look, lazy)]


def trailing_flops(m: int, n: int, lazy: int = 128) -> float:
    """Algorithmic flops of the trailing updates of one sweep of m rows (syntax.py:123): the sum over lazy blocks of
    2 m (b1 - b0) (n - b1)."""
    return float(sum(2 * m * (min(b0 + lazy, n) - b0) * (n - min(b0 + lazy, n)) for b0 in range(0, n, lazy)))


def causal_softmax(scores: torch.Tensor, scale: float, out: torch.Tensor | None = None) -> torch.Tensor:
    """bf16 probabilities of bf16 attention scores [..., T, T] (rows: sequence, head, query): the causal mask, the
    scale and a float32 softmax in one pass (lamq_causal_softmax_bf16). out may be scores itself."""
    need(scores, torch.bfloat16, "scores")
    T = scores.shape[-1]
    if scores.dim() < 2 or scores.shape[-2] != T or not scores.is_contiguous():
        raise ValueError("scores must be a contiguous [..., T, T] tensor")
    out = torch.empty_like(scores) if out is None else out
    need(out, torch.bfloat16, "out")
    if out.shape != scores.shape or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor of the scores' shape")
    rows = scores.numel() // T
    check(lib().lamq_causal_softmax_bf16(ptr(scores), ptr(out), rows, T, T, T, float(scale), stream(scores.device)),
          "causal_softmax")
    return out


def swiglu(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """silu(a) * b for contiguous bf16 a, b of one shape, rounded to bf16 after the silu and after the product, as
    the unfused chain rounds (lamq_swiglu_bf16)."""
    need(a, torch.bfloat16, "a")
    need(b, torch.bfloat16, "b")
    if a.shape != b.shape or not a.is_contiguous() or not b.is_contiguous() or a.numel() % 8:
        raise ValueError("a and b must be contiguous tensors of one shape, a multiple of 8 elements")
    y = torch.empty_like(a)
    check(lib().lamq_swiglu_bf16(ptr(a), ptr(b), ptr(y), a.numel(), stream(a.device)), "swiglu")
    return y


def rms_norm(x: torch.Tensor, g: torch.Tensor, eps: float, pad: int = 0) -> torch.Tensor:
    """bf16(bf16(x rsqrt(mean(x^2) + eps)) g) over the last dim of a bf16 x (float32 inside), one pass
    (lamq_rms_norm_bf16). x's rows may be strided (the last dim contiguous, one row stride); returns a new tensor of
    x's shape, contiguous, or with `pad` > 0 (a multiple of 8) a view of rows n + pad elements apart (row_pad)."""
    need(x, torch.bfloat16, "x")
    need(g, torch.bfloat16, "g", 1)
    n = x.shape[-1]
    if g.numel() != n:
        raise ValueError("g must have the last dim of x")
    if pad < 0 or pad % 8:
        raise ValueError("pad must be a non-negative multiple of 8")
    X = x.reshape(-1, n)
    if X.dim() == 2 and X.shape[0] > 1 and X.stride(1) != 1:
        raise ValueError("x must have a contiguous last dim")
    y = torch.empty(*x.shape[:-1], n + pad, dtype=x.dtype, device=x.device)[..., :n]
    check(lib().lamq_rms_norm_bf16(ptr(X), X.shape[0], n, X.stride(0) if X.shape[0] > 1 else n, ptr(g.contiguous()),
                                   ptr(y), n + pad, float(eps), stream(x.device)), "rms_norm")
    return y


def rms_norm_rope(x: torch.Tensor, g: torch.Tensor, eps: float, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """The per-head RMSNorm of q or k and the rotary embedding after it, one pass (lamq_rms_norm_rope_bf16): for x
    [B, T, heads, 128] bf16 (rows of 128 one stride apart) and cos, sin [T, 128] bf16, y = rms_norm(x, g, eps) then
    y * cos + rotate_half(y) * sin with the bf16 roundings of that chain (transformers' apply_rotary_pos_emb).
    Returns a new contiguous [B, T, heads, 128] tensor."""
    need(x, torch.bfloat16, "x", 4)
    need(g, torch.bfloat16, "g", 1)
    B, T, heads, n = x.shape
    if n != 128 or g.numel() != n:
        raise ValueError("x must be [B, T, heads, 128] and g [128]")
    for t, nm in ((cos, "cos"), (sin, "sin")):
        need(t, torch.bfloat16, nm, 2)
        if t.shape != (T, n) or t.stride(1) != 1:
            raise ValueError(f"{nm} must be [T, 128] with a contiguous last dim")
    if cos.stride(0) != sin.stride(0):
        raise ValueError("cos and sin must share one row stride")
    X = x.reshape(-1, n)
    if X.stride(1) != 1:
        raise ValueError("x must have a contiguous last dim")
    y = torch.empty(B, T, heads, n, dtype=x.dtype, device=x.device)
    rows = X.shape[0]
    check(lib().lamq_rms_norm_rope_bf16(ptr(X), rows, n, X.stride(0) if rows > 1 else n, ptr(g.contiguous()), ptr(cos),
                                        ptr(sin), cos.stride(0), heads, T, ptr(y), n, float(eps), stream(x.device)),
          "rms_norm_rope")
    return y


def row_pad(n: int) -> int:
    """Elements of padding after each row of bf16 activations whose Gram (lamq_hessian_accum, lamq_cross_gram) is
    taken: 192 at n = 2,560, whose 5,120-byte rows measured 15-20% slower in the Gram kernels than 5,504-byte ones (a
    channel effect of that stride); 0 elsewhere (no difference at n = 9,728)."""
    return 192 if n == 2560 else 0


def attention_causal(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """Causal grouped-query attention, fused (lamq_attention_causal_bf16): q [B, H, T, 128], k and v [B, Hkv, T, 128]
    bf16, any strides with the head dim contiguous; query head h reads key/value head h // (H / Hkv). Returns out
    [B, H, T, 128] bf16, by default a view of a [B, T, H, 128] buffer (the o_proj input's layout)."""
    for t, nm in ((q, "q"), (k, "k"), (v, "v")):
        need(t, torch.bfloat16, nm, 4)
        if t.stride(3) != 1:
            raise ValueError(f"{nm} must have a contiguous head dim")
    B, H, T, D = q.shape
    Hkv = k.shape[1]
    if k.shape != (B, Hkv, T, D) or v.shape != k.shape or H % Hkv:
        raise ValueError("k and v must be [B, Hkv, T, D] with Hkv dividing q's heads")
    if out is None:
        out = torch.empty(B, T, H, D, dtype=q.dtype, device=q.device).transpose(1, 2)
    need(out, torch.bfloat16, "out", 4)
    if out.shape != q.shape or out.stride(3) != 1:
        raise ValueError("out must be [B, H, T, D] with a contiguous head dim")
    check(lib().lamq_attention_causal_bf16(ptr(q), q.stride(0), q.stride(1), q.stride(2), ptr(k), k.stride(0),
                                           k.stride(1), k.stride(2), ptr(v), v.stride(0), v.stride(1), v.stride(2),
                                           ptr(out), out.stride(0), out.stride(1), out.stride(2), B, H, Hkv, T, D,
                                           float(scale), stream(q.device)), "attention_causal")
    return out


class EventLog(dict):
    """key -> list of (start, end) torch.cuda.Event pairs. lead_cycles > 0: before each span's start event, a GPU spin
    of that many cycles (torch.cuda._sleep) keeps the stream busy while the host enqueues the span, so that a span
    times its kernel and not the host's launch latency where the host, not the GPU, sets the pace."""

    lead_cycles = 0


def _lead(events):
    if getattr(events, "lead_cycles", 0):
        torch.cuda._sleep(int(events.lead_cycles))


class KernelTimer:
    """Event pairs recorded on the current stream around launches, by key, with the algorithmic work (flops, ops or
    bytes) each span does. events[key] is the list of (start, end) torch.cuda.Event pairs (the sweeps append their
    per-launch pairs under "block" and "trailing" to the same log). lead_cycles: see EventLog."""

    def __init__(self, lead_cycles: int = 0):
        self.events = EventLog()
        self.events.lead_cycles = int(lead_cycles)
        self.work: dict = {}

    @contextlib.contextmanager
    def span(self, key: str, work: float = 0.0):
        _lead(self.events)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        yield
        b.record()
        self.events.setdefault(key, []).append((a, b))
        self.work[key] = self.work.get(key, 0.0) + float(work)

    def add_work(self, key: str, work: float):
        self.work[key] = self.work.get(key, 0.0) + float(work)

    def ms(self, key: str) -> float:
        """Summed duration of the key's spans in ms (synchronise first)."""
        return sum(event_ms(self.events, key))

    def launches(self, key: str) -> int:
        return len(self.events.get(key, []))


def span(timer: KernelTimer | None, key: str, work: float = 0.0):
    """timer.span(key, work), or nothing without a timer."""
    return contextlib.nullcontext() if timer is None else timer.span(key, work)


def event_ms(events: dict, key: str) -> list[float]:
    """Durations in ms of the launches recorded under `key` (synchronise first)."""
    return [a.elapsed_time(b) for a, b in events.get(key, [])]


def ldlq_scalar(T0: torch.Tensor, U: torch.Tensor, levels: torch.Tensor, mode: int = 0, S: torch.Tensor | None = None,
                lazy: int = 128, dead: torch.Tensor | None = None, events: dict | None = None) -> torch.Tensor:
    """Level indices [m, n] int32 of the width-1 LDLQ onto `levels` (mode 0: T0 = X/S and the first argmin of the
    squared distance; mode 1: T0 = X and bucketize(t/S) on midpoints, q*S). events: as ldlq_trellis's ("block" the
    scalar block kernel, "trailing" the products)."""
    need(T0, torch.float64, "T0", 2)
    need(U, torch.float64, "U", 2)
    need(levels, torch.float64, "levels", 1)
    if mode == 1:
        need(S, torch.float64, "S", 1)
    m, n = T0.shape
    if lazy > 128:
        raise NotImplementedError("the width-1 block kernel keeps at most 128 columns of a row in registers")
    T = T0.clone(memory_format=torch.contiguous_format)
    dev = T0.device
    s = stream(dev)
    if dead is not None:
        dd = dead.to(device=dev, dtype=torch.uint8).contiguous()
        check(lib().lamq_zero_columns(ptr(T), m, n, n, ptr(dd), s), "zero_columns")
    idx = torch.empty(m, n, dtype=torch.int32, device=dev)
    outer = _outer_run(lazy)
    Z = torch.empty(m, outer, dtype=torch.float64, device=dev)
    for B0 in range(0, n, outer):
        B1 = min(B0 + outer, n)
        for b0 in range(B0, B1, lazy):
            b1 = min(b0 + lazy, n)
            zb = Z[:, b0 - B0 :]
            ev = _event_pair(events, "block")
            check(lib().lamq_ldlq_scalar_block(ptr(T), m, n, n, ptr(U), ld(U), ptr(S), ptr(levels), levels.numel(), mode,
                                               b0, b1, ptr(idx), n, ptr(zb), outer, s), "ldlq_scalar_block")
            _event_end(ev)
            _refit_run(T, U, zb, b0, b1, B1, 0, events)
        _refit_rest(T, U, Z, B0, B1, 0, events)
    return idx


def ldlq_multirate(X: torch.Tensor, U: torch.Tensor | None, tables: torch.Tensor, weights: torch.Tensor,
                   lazy: int = 128, dead: torch.Tensor | None = None, events: dict | None = None) -> torch.Tensor:
    """Indices [m, n] int32 of the width-1 sweep of X (units of the row scale) for R rates at once
    (nested.py:104-147): per entry the first argmin over the table index of sum_r w_r (t_r - tables[r, i])^2, each rate's
    copy of the row refit for its own value under U (lamq_ldlq_multirate_block over X.repeat(R, 1)); U None: every
    column alone."""
    need(X, torch.float64, "X", 2)
    need(tables, torch.float64, "tables", 2)
    need(weights, torch.float64, "weights", 1)
    if U is not None:
        need(U, torch.float64, "U", 2)
    R, K = tables.shape
    if weights.numel() != R:
        raise ValueError("one weight per rate")
    if lazy > 128:
        raise NotImplementedError("the width-1 block kernel keeps at most 128 columns of a row in registers")
    m, n = X.shape
    dev = X.device
    s = stream(dev)
    T = X.repeat(R, 1).contiguous()
    if dead is not None and U is not None:
        dd = dead.to(device=dev, dtype=torch.uint8).contiguous()
        check(lib().lamq_zero_columns(ptr(T), R * m, n, n, ptr(dd), s), "zero_columns")
    idx = torch.empty(m, n, dtype=torch.int32, device=dev)
    tab = tables.contiguous()
    wts = weights.contiguous()
    if U is None:
        for b0 in range(0, n, lazy):
            b1 = min(b0 + lazy, n)
            check(lib().lamq_ldlq_multirate_block(ptr(T), m, n, n, None, n, ptr(tab), R, K, ptr(wts), b0, b1, ptr(idx), n,
                                                  None, 1, s), "ldlq_multirate_block")
        return idx
    outer = _outer_run(lazy)
    Z = torch.empty(R * m, outer, dtype=torch.float64, device=dev)
    for B0 in range(0, n, outer):
        B1 = min(B0 + outer, n)
        for b0 in range(B0, B1, lazy):
            b1 = min(b0 + lazy, n)
            zb = Z[:, b0 - B0 :]
            ev = _event_pair(events, "block")
            check(lib().lamq_ldlq_multirate_block(ptr(T), m, n, n, ptr(U), ld(U), ptr(tab), R, K, ptr(wts), b0, b1,
                                                  ptr(idx), n, ptr(zb), outer, s), "ldlq_multirate_block")
            _event_end(ev)
            _refit_run(T, U, zb, b0, b1, B1, 0, events)
        _refit_rest(T, U, Z, B0, B1, 0, events)
    return idx


def refit_step(T: torch.Tensor, U: torch.Tensor, Q: torch.Tensor, j: int, b0: int, b1: int, Z: torch.Tensor):
    """E = T[:, j:j+w] - Q, z = E U_BB^-1, T[:, j+w:b1] -= z U[j:j+w, j+w:b1], Z[:, j-b0:j-b0+w] = z (in place)."""
    need(T, torch.float64, "T", 2)
    need(U, torch.float64, "U", 2)
    need(Q, torch.float64, "Q", 2)
    need(Z, torch.float64, "Z", 2)
    m, n = T.shape
    w = Q.shape[1]
    check(lib().lamq_refit_step(ptr(T), m, n, ld(T), ptr(U), ld(U), ptr(Q), ld(Q), j, w, b0, b1, ptr(Z), ld(Z),
                                stream(T.device)), "refit_step")
    return T


def shaping_feedback(V: torch.Tensor, block: int) -> torch.Tensor:
    """The packed row-block feedback M_q = V[a:b, a:b]^-1 V[a:b, b:] of output shaping (nested.py:126-127), V the
    upper factor of the damped output sensitivity (lamq_shaping_feedback)."""
    need(V, torch.float64, "V", 2)
    m = V.shape[0]
    M = torch.empty(max(1, lib().lamq_shaping_feedback_size(m, block) // 8), dtype=torch.float64, device=V.device)
    check(lib().lamq_shaping_feedback(ptr(V), m, ld(V), block, ptr(M), stream(V.device)), "shaping_feedback")
    return M


def shaped_column(T: torch.Tensor, j: int, M: torch.Tensor, block: int, levels: torch.Tensor, idx: torch.Tensor,
                  Q: torch.Tensor) -> torch.Tensor:
    """Column j of T settled row block by row block under the feedback M (lamq_ldlq_shaped_column): its indices into
    idx[:, j], its levels into Q [m] (returned); T is only read."""
    need(T, torch.float64, "T", 2)
    need(idx, torch.int32, "idx", 2)
    m, n = T.shape
    lv = levels.to(device=T.device, dtype=torch.float64).contiguous()
    check(lib().lamq_ldlq_shaped_column(ptr(T), m, n, ld(T), j, ptr(M), block, ptr(lv), lv.numel(), ptr(idx), ld(idx),
                                        ptr(Q), stream(T.device)), "ldlq_shaped_column")
    return Q


def zero_columns(T: torch.Tensor, dead: torch.Tensor):
    need(T, torch.float64, "T", 2)
    m, n = T.shape
    dd = dead.to(device=T.device, dtype=torch.uint8).contiguous()
    check(lib().lamq_zero_columns(ptr(T), m, n, ld(T), ptr(dd), stream(T.device)), "zero_columns")
    return T


def trailing_update(T: torch.Tensor, Z: torch.Tensor, U: torch.Tensor, b0: int, b1: int):
    """T[:, b1:] -= Z @ U[b0:b1, b1:] in place (syntax.py:123)."""
    need(T, torch.float64, "T", 2)
    need(Z, torch.float64, "Z", 2)
    need(U, torch.float64, "U", 2)
    m, n = T.shape
    check(lib().lamq_trailing_update_f64(ptr(T), m, n, ld(T), ptr(Z), ld(Z), ptr(U), ld(U), b0, b1, stream(T.device)),
          "trailing_update")
    return T


def gemm_sub(C: torch.Tensor, A: torch.Tensor, B: torch.Tensor, transb: bool = False, tri: int = 0) -> torch.Tensor:
    """C -= A @ op(B) in place (op(B) = B.T when transb), fp64 on MFMA; tri = 1 / 2 when op(B) is lower / upper
    triangular (its zero part is skipped)."""
    need(C, torch.float64, "C", 2)
    need(A, torch.float64, "A", 2)
    need(B, torch.float64, "B", 2)
    M, N = C.shape
    K = A.shape[1]
    if A.shape[0] != M or (B.shape != (N, K) if transb else B.shape != (K, N)):
        raise ValueError("gemm_sub: shapes do not agree")
    check(lib().lamq_gemm_sub_f64(ptr(C), ld(C), ptr(A), ld(A), ptr(B), ld(B), M, N, K, 1 if transb else 0, int(tri),
                                  stream(C.device)), "gemm_sub")
    return C


# ----------------------------------------------------------------------------- statistics


MAX_WEIGHT_CLASSES = 8


def _tiled(X: torch.Tensor) -> bool:
    """X meets the 256-tile Gram kernel's layout: 16-byte rows and base."""
    n = X.shape[1]
    return n % 8 == 0 and ld(X) % 8 == 0 and X.data_ptr() % 16 == 0


_CLASS_CACHE: dict = {}


def weight_classes(w: torch.Tensor, include_zero: bool = False):
    """[(weight, int32 row indices)] for the distinct values of w (the zero class only with include_zero) when there
    are at most MAX_WEIGHT_CLASSES of them, else None. Finding them synchronises with the host, so the last few
    results are kept, keyed by the tensor's storage, shape and version counter (an in-place change of w bumps the
    version)."""
    key = (w.data_ptr(), tuple(w.shape), w.dtype, str(w.device), w._version, include_zero)
    hit = _CLASS_CACHE.get(key)
    if hit is not None and hit[0] is w:
        return hit[1]
    vals = torch.unique(w)
    if vals.numel() > MAX_WEIGHT_CLASSES:
        out = None
    else:
        out = []
        for v in vals.cpu().tolist():
            if v != 0.0 or include_zero:
                out.append((v, (w == v).nonzero().flatten().to(torch.int32)))
    if len(_CLASS_CACHE) >= 16:
        _CLASS_CACHE.pop(next(iter(_CLASS_CACHE)))
    _CLASS_CACHE[key] = (w, out)
    return out


def hessian_accum(H: torch.Tensor, X: torch.Tensor, w: torch.Tensor | None = None, scale: float = 1.0,
                  classes: list | None = None) -> torch.Tensor:
    """H (float32 [n, n], lower triangle) += scale * X^T diag(w) X for bf16 X [N, n]. Weights with few distinct
    values are taken class by class through the unweighted kernel (exact products): the most frequent weight w0
    over all tokens (contiguous), then (v - w0) over each other class's rows (gathered in the kernel). Other
    weights use the hi/lo split. classes: weight_classes(w, include_zero=True), if the caller has it already; classes
    that leave tokens out (weight_classes without the zero class) are taken one by one, each over its own rows, so a
    token outside every class counts with weight 0."""
    need(H, torch.float32, "H", 2)
    need(X, torch.bfloat16, "X", 2)
    N, n = X.shape
    wv = None
    if w is not None:
        wv = w.to(device=X.device, dtype=torch.float32).contiguous()
        if classes is None and _tiled(X):
            classes = weight_classes(wv, include_zero=True)
        if classes is not None and _tiled(X):
            base = 0.0
            if sum(rows.numel() for _, rows in classes) == N:  # every token in a class: a contiguous base pass
                base, _ = max(classes, key=lambda c: c[1].numel())
            if base != 0.0:
                nbytes = lib().lamq_gram_workspace_size(N, n, 1)
                ws = workspace(nbytes, X.device)
                check(lib().lamq_hessian_accum(ptr(X), N, n, ld(X), None, float(scale * base), ptr(H), ld(H), ptr(ws),
                                               nbytes, stream(X.device)), "hessian_accum")
            for v, rows in classes:
                if v == base or rows.numel() == 0:
                    continue
                m = rows.numel()
                nbytes = lib().lamq_gram_workspace_size(m, n, 1)
                ws = workspace(nbytes, X.device)
                check(lib().lamq_hessian_accum_rows(ptr(X), ptr(rows), m, n, ld(X), float(scale * (v - base)), ptr(H),
                                                    ld(H), ptr(ws), nbytes, stream(X.device)), "hessian_accum_rows")
            return H
    nbytes = lib().lamq_gram_workspace_size(N, n, 1)
    ws = workspace(nbytes, X.device)
    check(lib().lamq_hessian_accum(ptr(X), N, n, ld(X), ptr(wv), float(scale), ptr(H), ld(H), ptr(ws), nbytes,
                                   stream(X.device)), "hessian_accum")
    return H


def hessian_finalize(H: torch.Tensor, ntok: float, want64: bool = True):
    need(H, torch.float32, "H", 2)
    n = H.shape[0]
    H64 = torch.empty(n, n, dtype=torch.float64, device=H.device) if want64 else None
    check(lib().lamq_hessian_finalize(ptr(H), n, ld(H), float(ntok), ptr(H64), n, stream(H.device)), "hessian_finalize")
    return H64 if want64 else H


def hessian(X: torch.Tensor, w: torch.Tensor | None = None) -> torch.Tensor:
    """H = (1/N) X^T diag(w) X as float64 [n, n] from bf16 activations [N, n] (quantize.py:1465,1470)."""
    N, n = X.shape
    H = torch.zeros(n, n, dtype=torch.float32, device=X.device)
    hessian_accum(H, X, w)
    return hessian_finalize(H, float(N))


def cross_gram_accum(D: torch.Tensor, Xr: torch.Tensor, Xq: torch.Tensor, w: torch.Tensor | None = None,
                     scale: float = 1.0, classes: list | None = None) -> torch.Tensor:
    """D (float32 [n, n]) += scale * Xr^T diag(w) Xq (quantize.py:1457). Weights with few distinct values go class by
    class through the unweighted kernel, as in hessian_accum: the most frequent weight w0 over all tokens
    (contiguous), then (v - w0) over each other class's rows (gathered in the kernel). classes:
    weight_classes(w, include_zero=True), if the caller has it already (classes that leave rows out are taken one by
    one, each over its own rows)."""
    need(D, torch.float32, "D", 2)
    need(Xr, torch.bfloat16, "Xr", 2)
    need(Xq, torch.bfloat16, "Xq", 2)
    if Xr.shape != Xq.shape or ld(Xr) != ld(Xq):
        raise ValueError("Xr and Xq must have the same shape and row stride")
    N, n = Xr.shape
    wv = None if w is None else w.to(device=Xr.device, dtype=torch.float32).contiguous()
    if wv is not None and _tiled(Xr) and _tiled(Xq):
        if classes is None:
            classes = weight_classes(wv, include_zero=True)
        if classes is not None:
            base = 0.0
            if sum(rows.numel() for _, rows in classes) == N:  # every token in a class: a contiguous base pass
                base, _ = max(classes, key=lambda c: c[1].numel())
            if base != 0.0:
                nbytes = lib().lamq_gram_workspace_size(N, n, 0)
                ws = workspace(nbytes, Xr.device)
                check(lib().lamq_cross_gram(ptr(Xr), ptr(Xq), N, n, ld(Xr), None, float(scale * base), ptr(D), ld(D),
                                            ptr(ws), nbytes, stream(Xr.device)), "cross_gram")
            for v, rows in classes:  # the other classes' rows are gathered inside the kernel, no copies
                if v == base or rows.numel() == 0:
                    continue
                nbytes = lib().lamq_gram_workspace_size(rows.numel(), n, 0)
                ws = workspace(nbytes, Xr.device)
                check(lib().lamq_cross_gram_rows(ptr(Xr), ptr(Xq), ptr(rows), rows.numel(), n, ld(Xr),
                                                 float(scale * (v - base)), ptr(D), ld(D), ptr(ws), nbytes,
                                                 stream(Xr.device)), "cross_gram_rows")
            return D
    nbytes = lib().lamq_gram_workspace_size(N, n, 0)
    ws = workspace(nbytes, Xr.device)
    check(lib().lamq_cross_gram(ptr(Xr), ptr(Xq), N, n, ld(Xr), ptr(wv), float(scale), ptr(D), ld(D), ptr(ws), nbytes,
                                stream(Xr.device)), "cross_gram")
    return D


# ----------------------------------------------------------------------------- KL (compiler.py:177-188)


def kl_rows(ref: torch.Tensor, q: torch.Tensor, w: torch.Tensor | None = None):
    """(kl [T] float32, sums [2] float64 = (sum w kl, sum w)) for logits [T, V], both bf16 (lamq_kl_rows) or both
    float32 (lamq_kl_rows_f32)."""
    dt = ref.dtype if ref.dtype in (torch.bfloat16, torch.float32) else torch.bfloat16
    need(ref, dt, "ref", 2)
    need(q, dt, "q", 2)
    if ref.shape != q.shape:
        raise ValueError("ref and q must have the same shape")
    T, V = ref.shape
    wv = None if w is None else w.to(device=ref.device, dtype=torch.float32).contiguous()
    kl = torch.empty(T, dtype=torch.float32, device=ref.device)
    sums = torch.empty(2, dtype=torch.float64, device=ref.device)
    nbytes = lib().lamq_kl_workspace_size(T)
    ws = workspace(nbytes, ref.device)
    fn = lib().lamq_kl_rows if dt == torch.bfloat16 else lib().lamq_kl_rows_f32
    check(fn(ptr(ref), ptr(q), T, V, ld(ref), ld(q), ptr(wv), ptr(kl), ptr(sums), ptr(ws), nbytes, stream(ref.device)),
          "kl_rows")
    return kl, sums


KL_NOALLOC_MAX_T = 65536  # LAMQ_KL_NOALLOC_MAX_T


def kl_rows_noalloc(ref: torch.Tensor, q: torch.Tensor, kl: torch.Tensor, sums: torch.Tensor | None,
                    w: torch.Tensor | None = None):
    """kl_rows into caller-owned outputs (kl [T] float32, sums [2] float64 or None) through lamq_kl_rows_noalloc,
    which allocates nothing: its partials live in a static per-device array of KL_NOALLOC_MAX_T tokens, shared by
    every call on that GPU (calls that overlap on one GPU race). w, if given, must already be a contiguous float32
    tensor on the device. T > KL_NOALLOC_MAX_T raises ValueError before any launch."""
    need(ref, torch.bfloat16, "ref", 2)
    need(q, torch.bfloat16, "q", 2)
    need(kl, torch.float32, "kl", 1)
    if ref.shape != q.shape or kl.numel() != ref.shape[0]:
        raise ValueError("ref and q must have the same shape and kl one entry per row")
    T, V = ref.shape
    if T > KL_NOALLOC_MAX_T:
        raise ValueError(f"kl_rows_noalloc takes at most {KL_NOALLOC_MAX_T} tokens per call (got {T})")
    if sums is not None:
        need(sums, torch.float64, "sums", 1)
        if sums.numel() < 2:
            raise ValueError("sums must hold two float64 values")
    if w is not None:
        need(w, torch.float32, "w", 1)
        if w.numel() != T:
            raise ValueError("one weight per token")
    check(lib().lamq_kl_rows_noalloc(ptr(ref), ptr(q), T, V, ld(ref), ld(q), ptr(w), ptr(kl), ptr(sums),
                                     stream(ref.device)), "kl_rows_noalloc")
    return kl, sums


# ----------------------------------------------------------------------------- packing (compiler_artifact.py:276-284)


def pack_trellis(states: torch.Tensor, k: int, L: int = 12, check_paths: bool = True):
    """int32 tensor holding the uint32 code words [m, ceil(n/32)*k] of row-trellis states. With check_paths a row
    that is not a path from state 0 raises ValueError (one host synchronisation); without it (codes, bad) is
    returned, bad a device flag."""
    need(states, torch.int32, "states", 2)
    m, n = states.shape
    words = (n + 31) // 32 * k
    codes = torch.empty(m, words, dtype=torch.int32, device=states.device)
    bad = torch.zeros(1, dtype=torch.int32, device=states.device)
    check(lib().lamq_pack_trellis(ptr(states), m, n, ld(states), k, L, ptr(codes), words, ptr(bad), stream(states.device)),
          "pack_trellis")
    if not check_paths:
        return codes, bad
    if int(bad.item()):
        raise ValueError("states are not a row trellis from zero")
    return codes


def pack_codes(src: torch.Tensor, k: int, rows: torch.Tensor | None = None, base: int = 0, L: int = 12,
               trellis: bool = True, out: torch.Tensor | None = None, bad: torch.Tensor | None = None):
    """The code words [m, ceil(n/32)*k] (an int32 tensor holding uint32 bits) of rows `rows` (int64 on the device,
    None for all rows) of the int32 code array src, minus `base`: row-trellis states (trellis) or scalar symbols.
    Returns (codes, bad): bad an int32 device flag, nonzero if a row was not a path from state 0 (or a symbol was
    outside [0, 2^k)). Several calls may share one `bad` flag; nothing synchronises."""
    need(src, torch.int32, "src", 2)
    nsrc, n = src.shape
    if rows is not None:
        if rows.dtype != torch.int64 or rows.device != src.device or rows.dim() != 1:
            raise ValueError("rows must be a 1-d int64 tensor on the device of src")
        rows = rows.contiguous()
    m = nsrc if rows is None else rows.shape[0]
    words = (n + 31) // 32 * k
    if out is None:
        out = torch.empty(m, words, dtype=torch.int32, device=src.device)
    elif out.shape != (m, words) or out.dtype != torch.int32 or out.stride(1) != 1:
        raise ValueError("out must be an int32 [m, ceil(n/32)*k] tensor with unit column stride")
    if bad is None:
        bad = torch.zeros(1, dtype=torch.int32, device=src.device)
    check(lib().lamq_pack_codes(ptr(src), ld(src), nsrc, ptr(rows), m, n, int(base), k, L, 1 if trellis else 0, ptr(out),
                                out.stride(0), ptr(bad), stream(src.device)), "pack_codes")
    return out, bad


def pack_codes_groups(items: list, L: int = 12, trellis: bool = True, bad: torch.Tensor | None = None):
    """pack_codes for many row groups in one launch (lamq_pack_codes_groups): items are (src, k, rows, base) with
    pack_codes's meanings, every src of the same width n and on one device. Returns ([codes of each item], bad), each
    item's words those pack_codes gives for it alone (an empty group's: no rows, nothing launched for it). Nothing
    synchronises."""
    if not items:
        raise ValueError("no groups to pack")
    n = items[0][0].shape[1]
    dev = items[0][0].device
    descs = (_abi.PackGroup * len(items))()
    outs, count = [], 0
    for src, k, rows, base in items:
        need(src, torch.int32, "src", 2)
        if src.shape[1] != n or src.device != dev:
            raise ValueError("every group's source must have the same width and device")
        if rows is not None:
            if rows.dtype != torch.int64 or rows.device != dev or rows.dim() != 1 or not rows.is_contiguous():
                raise ValueError("rows must be a contiguous 1-d int64 tensor on the device of src")
        m = src.shape[0] if rows is None else rows.shape[0]
        out = torch.empty(m, (n + 31) // 32 * k, dtype=torch.int32, device=dev)
        outs.append(out)
        if m == 0:
            continue
        d = descs[count]
        d.src, d.ld, d.src_rows, d.rows, d.m = ptr(src), ld(src), src.shape[0], ptr(rows), m
        d.base, d.k, d.codes, d.ldc = int(base), int(k), ptr(out), out.stride(0)
        count += 1
    if bad is None:
        bad = torch.zeros(1, dtype=torch.int32, device=dev)
    check(lib().lamq_pack_codes_groups(ctypes.addressof(descs), count, n, L, 1 if trellis else 0, ptr(bad),
                                       stream(dev)), "pack_codes_groups")
    return outs, bad
