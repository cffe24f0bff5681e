"""Block LDL factorisation and the LDLQ error-feedback traversal on the GPU
(reference: exl3_quant/ldlq.py).

``block_ldl`` factors the (Hadamard-rotated, damped) Hessian H = L L^T with a
blocked Cholesky (``cholesky_ex``: diagonal blocks factored by a HIP kernel,
panel updates and solves as GEMM-class library calls), inverts every 16x16
diagonal block in one batched call and folds the inverses into their block
columns with one batched GEMM; the diagonal blocks become identities.

``ldlq`` quantises a (k, n) weight bottom-up: spans of ``buf_size_k`` rows
from the last, 16-row blocks inside a span from the last. Each block's rows
get the compensation of the rows already quantised below it in the span
(``addmm`` against the strictly lower slice of L) plus the span-level
feedback ``prod_cache``; the 16 x n rows become n / 16 tiles in tensor-core
order, go through the tile encoder (the HIP encoder, tiles staying in HBM),
and the reconstruction is un-permuted into ``weight_q`` while the states stay
in tensor-core order. After a span its residual is propagated into
``prod_cache`` for the spans above. All of it runs on the weight's device.

A traversal is a chain of n / 16-tile encoder calls (256 tiles for a 4096
wide projection: one workgroup per CU, half the encoder's occupancy).
``ldlq_lockstep`` walks independent projections side by side and encodes
several of their blocks per call (``lockstep_schedule`` balances the calls).
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Callable, List, Optional, Sequence, Tuple

import torch

from .tile_encoder import TileEncoder, make_gpu_tile_encoder, make_xpu_tile_encoder
from .trellis_format import tensor_core_perm, tensor_core_perm_inv

DEFAULT_BLOCK_SIZE = 16
DEFAULT_SIGMA_REG = 0.025
DEFAULT_MAX_RETRIES = 10
DEFAULT_BUF_SIZE_K = 128

__all__ = ["DEFAULT_BLOCK_SIZE", "DEFAULT_SIGMA_REG", "DEFAULT_MAX_RETRIES", "DEFAULT_BUF_SIZE_K",
           "BlockLDLResult", "cholesky_ex", "block_ldl", "LDLQResult", "ldlq", "ldlq_lockstep",
           "lockstep_schedule", "TileEncoder", "make_xpu_tile_encoder", "make_gpu_tile_encoder"]


@dataclass(frozen=True)
class BlockLDLResult:
    """Folded factor and intermediates (ldlq.py:45-56)."""

    transformed: torch.Tensor
    cholesky: torch.Tensor
    block_inverses: torch.Tensor
    retries: int
    damping_applied: bool
    n: int
    block_size: int


def cholesky_ex(A: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Lower Cholesky factor of a symmetric positive-definite float32 GPU
    matrix and an int32 ``info``: 0, or the 1-based order of the first
    leading minor found not positive definite (``torch.linalg.cholesky_ex``'s
    contract; only the lower triangle of ``A`` is read, ``A`` is not
    modified).

    Left-looking and blocked by the HIP kernel's block order (128): panel j
    gets the product of the finished columns to its left subtracted (one
    GEMM, ``addmm_`` on the strided panel view), its diagonal block is
    factored in LDS by ``exl3_cholesky_diag_block`` and the rows below are
    solved against it (``solve_triangular``, a rocBLAS trsm). No host
    synchronisation: ``info`` stays on the device."""
    from ._native import cholesky_block_order, cholesky_diag_block
    if A.dim() != 2 or A.shape[0] != A.shape[1] or A.dtype != torch.float32:
        raise ValueError(f"cholesky_ex expects a square float32 matrix, got {A.dtype} "
                         f"{tuple(A.shape)}")
    if A.device.type != "cuda":
        raise ValueError("cholesky_ex runs on the GPU; move the matrix to a cuda device")
    n = A.shape[0]
    nb = cholesky_block_order()
    L = A.contiguous().clone()
    info = torch.zeros(1, dtype=torch.int32, device=A.device)
    for j0 in range(0, n, nb):
        j1 = min(n, j0 + nb)
        if j0 > 0:
            L[j0:, j0:j1].addmm_(L[j0:, :j0], L[j0:j1, :j0].T, beta=1.0, alpha=-1.0)
        cholesky_diag_block(L, j0, j1 - j0, info)
        if j1 < n:
            panel = L[j1:, j0:j1]
            panel.copy_(torch.linalg.solve_triangular(L[j0:j1, j0:j1].T, panel, upper=True,
                                                      left=False))
    return L.tril_(), info


def block_ldl(H: torch.Tensor, block_size: int = DEFAULT_BLOCK_SIZE,
              sigma_reg: float = DEFAULT_SIGMA_REG,
              max_retries: int = DEFAULT_MAX_RETRIES) -> BlockLDLResult:
    """Block-folded Cholesky factor consumed by :func:`ldlq` (ldlq.py:76-142).
    ``H`` is not modified; after a failed factorisation an internal copy is
    damped by 2 sigma_reg mean(diag) and factored again, up to
    ``max_retries`` times. The factorisation is :func:`cholesky_ex`; the
    diagonal 16 x 16 blocks of the factor are inverted in one batched call
    and folded into their block columns with one batched GEMM."""
    if H.dim() != 2 or H.shape[0] != H.shape[1]:
        raise ValueError(f"H must be a square 2-D tensor, got shape {tuple(H.shape)}")
    if H.dtype != torch.float32:
        raise ValueError(f"block_ldl requires float32, got {H.dtype}")
    if block_size <= 0 or block_size > H.shape[0] or H.shape[0] % block_size:
        raise ValueError(f"block_size {block_size} must be positive and divide {H.shape[0]}")
    if max_retries < 0:
        raise ValueError(f"max_retries must be non-negative, got {max_retries}")
    n = H.shape[0]
    work = H.clone()
    chol = None
    retries = 0
    for attempt in range(max_retries + 1):
        chol, info = cholesky_ex(work)
        if int(info.item()) == 0:
            retries = attempt
            break
        if attempt == max_retries:
            raise torch.linalg.LinAlgError(
                f"block_ldl: Cholesky failed after {max_retries} damping steps")
        work.diagonal().add_(2.0 * sigma_reg * work.diagonal().mean())
    m = n // block_size
    # The m diagonal blocks as a strided view: [b, r, c] = chol[b bs + r, b bs + c].
    diag_view = chol.view(m, block_size, m, block_size).diagonal(dim1=0, dim2=2)
    inverses = torch.linalg.inv(diag_view.permute(2, 0, 1).contiguous())
    # Column block b of the factor times its inverse: one batched GEMM.
    cols = chol.view(n, m, block_size).permute(1, 0, 2).contiguous()      # (m, n, bs)
    folded = torch.matmul(cols, inverses)                                  # (m, n, bs)
    transformed = folded.permute(1, 0, 2).reshape(n, n).contiguous()
    eye = torch.eye(block_size, dtype=H.dtype, device=H.device)
    transformed.view(m, block_size, m, block_size).diagonal(dim1=0, dim2=2).copy_(
        eye.unsqueeze(-1).expand(block_size, block_size, m))
    return BlockLDLResult(transformed=transformed, cholesky=chol, block_inverses=inverses,
                          retries=retries, damping_applied=retries > 0, n=n,
                          block_size=block_size)


@dataclass
class LDLQResult:
    """Quantised layer and its trellis states (ldlq.py:150-158)."""

    weight_q: torch.Tensor
    encoded: torch.Tensor
    tiles_k: int
    tiles_n: int
    buf_size_k: int
    encoder_seconds: float = 0.0
    encoder_calls: int = 0
    timings: dict = field(default_factory=dict)


def _as_int16_states(indices: torch.Tensor) -> torch.Tensor:
    """16-bit states in a signed int16 container, bit pattern kept (ldlq.py:147-160)."""
    if indices.dtype == torch.int16:
        return indices
    values = indices.to(torch.int64) & 0xFFFF
    return torch.where(values >= 0x8000, values - 0x10000, values).to(torch.int16)


class _Traversal:
    """One weight's bottom-up LDLQ walk, block by block.

    On a GPU the walk keeps E = W - Wq beside Wq: ``compensate(b)`` adds the
    feedback of the rows already quantised below block b in its span to the
    block's compensation rows (one GEMM), the HIP kernels
    ``exl3_ldlq_gather`` / ``exl3_ldlq_scatter`` form the encoder's tiles
    and write Wq, E and the states back for every block of a call at once,
    and ``span_feedback(b)`` propagates a finished span's residual into the
    compensation of the rows above it (one GEMM over those rows only: the
    factor is lower triangular and rows at or below the span are never read
    again). CPU tensors take the same steps as torch operations
    (``tiles`` / ``store``)."""

    def __init__(self, weight: torch.Tensor, L: torch.Tensor, buf_size_k: int):
        if weight.dim() != 2 or weight.dtype != torch.float32:
            raise ValueError(f"weight must be a 2-D float32 tensor, got {weight.dtype} "
                             f"{tuple(weight.shape)}")
        k, n = weight.shape
        if k % 16 != 0:
            raise ValueError(f"rows ({k}) must be a multiple of 16")
        if n % 128 != 0:
            raise ValueError(f"columns ({n}) must be a multiple of 128")
        if L.dim() != 2 or tuple(L.shape) != (k, k) or L.dtype != torch.float32:
            raise ValueError(f"L must be a float32 ({k}, {k}) tensor, got {L.dtype} "
                             f"{tuple(L.shape)}")
        if L.device != weight.device:
            raise ValueError(f"L and weight must be on the same device, got {L.device} / "
                             f"{weight.device}")
        buf_size_k = int(buf_size_k)
        if buf_size_k < 16 or buf_size_k % 16 != 0:
            raise ValueError(f"buf_size_k must be a positive multiple of 16, got {buf_size_k}")
        if n % buf_size_k != 0 or k % buf_size_k != 0:
            raise ValueError(f"rows ({k}) and columns ({n}) must be divisible by buf_size_k "
                             f"({buf_size_k})")
        device = weight.device
        self.on_gpu = device.type == "cuda"
        self.weight = weight.contiguous() if self.on_gpu else weight
        self.L, self.buf_size_k = L, buf_size_k
        self.tiles_k, self.tiles_n, self.n = k // 16, n // 16, n
        self.perm = torch.as_tensor(tensor_core_perm(), dtype=torch.long, device=device)
        self.inv_perm = torch.as_tensor(tensor_core_perm_inv(), dtype=torch.long, device=device)
        self.prod_cache = torch.zeros((k, n), dtype=torch.float32, device=device)
        self.weight_q = torch.zeros((k, n), dtype=torch.float32, device=device)
        self.err = torch.zeros((k, n), dtype=torch.float32, device=device) if self.on_gpu else None
        self.encoded = torch.zeros((k // 16, n // 16, 256), dtype=torch.int16, device=device)
        # (span start i, span end j, first row r0) in traversal order: spans
        # from the last, 16-row blocks inside a span from the last.
        self.blocks = [(j - buf_size_k, j, j - buf_size_k + bj - 16)
                       for j in range(k, 0, -buf_size_k) for bj in range(buf_size_k, 0, -16)]
        self.encoder_seconds = 0.0
        self.encoder_calls = 0

    # ------------------------------------------------------- GPU steps

    def compensate(self, b: int) -> None:
        i, j, r0 = self.blocks[b]
        r1 = r0 + 16
        if r1 < j:
            self.prod_cache[r0:r1].addmm_(self.L[r1:j, r0:r1].T, self.err[r1:j],
                                          alpha=1.0, beta=1.0)

    def span_feedback(self, b: int) -> None:
        i, j, r0 = self.blocks[b]
        if r0 == i and i > 0:
            self.prod_cache[:i].addmm_(self.L[i:j, :i].T, self.err[i:j], alpha=1.0, beta=1.0)

    def block_row(self, b: int, tile0: int, bases: Optional[tuple] = None) -> list:
        """The ``exl3_ldlq_block`` fields of block b at batch tile ``tile0``;
        ``bases`` = ``block_bases()``, when the caller has it."""
        _, _, r0 = self.blocks[b]
        row = r0 * self.n * 4
        w, comp, wq, err, states = bases if bases is not None else self.block_bases()
        return [w + row, comp + row, wq + row, err + row,
                states + (r0 // 16) * self.tiles_n * 256 * 2, self.n, tile0, 0]

    def block_bases(self) -> tuple:
        """Device addresses of W, the compensation rows, Wq, E and the states."""
        return (self.weight.data_ptr(), self.prod_cache.data_ptr(), self.weight_q.data_ptr(),
                self.err.data_ptr(), self.encoded.data_ptr())

    # ------------------------------------------------------- CPU steps

    def tiles(self, b: int) -> torch.Tensor:
        i, j, r0 = self.blocks[b]
        r1 = r0 + 16
        comp = self.prod_cache[r0:r1]
        if r1 < j:
            # Rows already quantised below, within this span.
            err = self.weight[r1:j] - self.weight_q[r1:j]
            comp.addmm_(self.L[r1:j, r0:r1].T, err, alpha=1.0, beta=1.0)
        rows = self.weight[r0:r1] + comp
        tiles = rows.reshape(16, self.tiles_n, 16).permute(1, 0, 2).reshape(self.tiles_n, 256)
        return tiles[:, self.perm].contiguous()

    def store(self, b: int, quant_w: torch.Tensor, quant_i: torch.Tensor) -> None:
        i, j, r0 = self.blocks[b]
        device = self.weight.device
        quant_w = quant_w.to(device=device, dtype=torch.float32)[:, self.inv_perm]
        self.weight_q[r0:r0 + 16] = (quant_w.reshape(self.tiles_n, 16, 16).permute(1, 0, 2)
                                     .reshape(16, self.n))
        self.encoded[r0 // 16] = _as_int16_states(quant_i.to(device=device))
        if r0 == i and i > 0:
            # Span residual into the feedback of the spans above.
            self.prod_cache[:i].addmm_(self.L[i:j, :i].T, self.weight[i:j] - self.weight_q[i:j],
                                       alpha=1.0, beta=1.0)

    def result(self) -> "LDLQResult":
        return LDLQResult(weight_q=self.weight_q, encoded=self.encoded, tiles_k=self.tiles_k,
                          tiles_n=self.tiles_n, buf_size_k=self.buf_size_k,
                          encoder_seconds=self.encoder_seconds,
                          encoder_calls=self.encoder_calls)


# Tiles one pass of the encoder runs at once on MI355X (256 CUs x two
# 1024-thread workgroups): the unit a lockstep call's size is rounded to.
LOCKSTEP_ROUND_TILES = 512


def lockstep_schedule(block_counts: Sequence[int], tiles_per_block: Sequence[int],
                      round_tiles: int = LOCKSTEP_ROUND_TILES) -> List[List[int]]:
    """The walks that advance one block in each encoder call of a lockstep
    traversal. There are max(block_counts) calls: the longest walk advances
    in every one. A call first takes every walk that must advance (as many
    blocks left as calls left), then the others, fewest spare calls first,
    while the call stays within the mean tiles per call rounded up to a
    multiple of ``round_tiles``. Walks keep their order inside a call. Every
    walk's blocks stay in order, so each result equals its own traversal."""
    if len(block_counts) != len(tiles_per_block):
        raise ValueError("block_counts and tiles_per_block differ in length")
    if not block_counts:
        return []
    calls = max(block_counts)
    total = sum(b * t for b, t in zip(block_counts, tiles_per_block))
    per_call = -(-total // calls)
    target = max(round_tiles, -(-per_call // round_tiles) * round_tiles)
    remaining = list(block_counts)
    schedule = []
    for c in range(calls):
        left = calls - c
        order = sorted((w for w in range(len(remaining)) if remaining[w] > 0),
                       key=lambda w: (left - remaining[w], w))
        load, members = 0, []
        for w in order:
            if remaining[w] == left or load + tiles_per_block[w] <= target:
                members.append(w)
                load += tiles_per_block[w]
        members.sort()
        for w in members:
            remaining[w] -= 1
        schedule.append(members)
    return schedule


def _block_table(walks: List[_Traversal], steps: List[List[Tuple[int, int]]]):
    """Device table of ``exl3_ldlq_block`` rows for every call, and each
    call's (first row, row count, tiles)."""
    import numpy as np
    for w in walks:
        for t in (w.weight, w.prod_cache, w.weight_q, w.err, w.encoded):
            if not t.is_contiguous():
                raise ValueError("LDLQ buffers must be contiguous")
    from ._native import check_ldlq_table
    bases = [w.block_bases() for w in walks]
    rows, spans = [], []
    for call in steps:
        tile0 = 0
        first = len(rows)
        for w, b in call:
            rows.append(walks[w].block_row(b, tile0, bases[w]))
            tile0 += walks[w].tiles_n
        spans.append((first, len(call), tile0))
    rows = np.asarray(rows, dtype=np.int64)
    # One vectorised check for the whole traversal: call by call it took
    # about 14 us of host time per call, all before the first call is queued.
    check_ldlq_table(rows, spans)
    table = torch.from_numpy(rows).to(walks[0].weight.device)
    return table, spans


class _Lane:
    """A set of walks whose blocks share encoder calls, as
    :func:`lockstep_schedule` assigns them, with its own encoder adapter and
    (on a GPU with several lanes) its own stream."""

    def __init__(self, walks: List[_Traversal], encode_tiles: TileEncoder,
                 synchronize: Optional[Callable[[], None]], stream=None,
                 time_calls: bool = True):
        self.walks, self.encode_tiles, self.synchronize = walks, encode_tiles, synchronize
        self.stream = stream
        schedule = lockstep_schedule([len(w.blocks) for w in walks], [w.tiles_n for w in walks])
        nxt = [0] * len(walks)
        self.steps = []
        for members in schedule:
            self.steps.append([(w, nxt[w]) for w in members])
            for w in members:
                nxt[w] += 1
        self.device = walks[0].weight.device
        self.fused = walks[0].on_gpu
        if self.fused:
            self.table, self.spans = _block_table(walks, self.steps)
        # Each timing event costs the stream about 5 us (a 256-tile call is
        # about 0.5 ms), so event timing is the caller's choice.
        self.use_events = time_calls and synchronize is None and self.fused
        self.pending = []      # (event pair, [(walk, tiles)]) read after the loop
        self.done = 0

    def issue(self) -> None:
        """Queue the lane's next encoder call and the steps around it."""
        from ._native import ldlq_gather, ldlq_scatter
        walks, call, device = self.walks, self.steps[self.done], self.device
        if self.fused:
            first, count, n_tiles = self.spans[self.done]
            rows = self.table[first:first + count]
            for w, b in call:
                walks[w].compensate(b)
            batch = torch.empty((n_tiles, 256), dtype=torch.float32, device=device)
            ldlq_gather(rows, batch)
        else:
            parts = [walks[w].tiles(b) for w, b in call]
            batch = parts[0] if len(parts) == 1 else torch.cat(parts)
        if self.use_events:
            ev0 = torch.cuda.Event(enable_timing=True)
            ev0.record()
        elif self.synchronize is not None:
            self.synchronize()
        t0 = time.perf_counter()
        quant_w, quant_i = self.encode_tiles(batch)
        if self.use_events:
            ev1 = torch.cuda.Event(enable_timing=True)
            ev1.record()
            self.pending.append(((ev0, ev1), [(walks[w], walks[w].tiles_n) for w, _ in call]))
        elif self.synchronize is not None or not self.fused:
            # Host wall time: the call is synchronised, or runs on the host.
            if self.synchronize is not None:
                self.synchronize()
            dt = time.perf_counter() - t0
            for w, _ in call:
                walks[w].encoder_seconds += dt * walks[w].tiles_n / batch.shape[0]
        if tuple(quant_w.shape) != (batch.shape[0], 256) or tuple(quant_i.shape) != (batch.shape[0], 256):
            raise ValueError("encode_tiles must return two (tiles_n, 256) tensors, got "
                             f"{tuple(quant_w.shape)} / {tuple(quant_i.shape)}")
        if self.fused:
            recon = quant_w.to(device=device, dtype=torch.float32).contiguous()
            idx = _as_int16_states(quant_i.to(device=device)).contiguous()
            ldlq_scatter(rows, recon, idx)
            for w, b in call:
                walks[w].span_feedback(b)
        else:
            off = 0
            for w, b in call:
                walk = walks[w]
                walk.store(b, quant_w[off:off + walk.tiles_n], quant_i[off:off + walk.tiles_n])
                off += walk.tiles_n
        for w, _ in call:
            walks[w].encoder_calls += 1
        self.done += 1

    def intervals(self, ref) -> List[Tuple[float, float]]:
        """Start and end of every encoder call, seconds after event ``ref``."""
        return [(ref.elapsed_time(ev0) / 1e3, ref.elapsed_time(ev1) / 1e3)
                for (ev0, ev1), _ in self.pending]

    def finish(self, scale: float = 1.0) -> None:
        """Credit each call's duration (times ``scale``) to its walks by
        tile share, then raise on NaN inputs the encoder counted."""
        if self.pending:
            self.pending[-1][0][1].synchronize()
            for (ev0, ev1), members in self.pending:
                dt = ev0.elapsed_time(ev1) / 1e3 * scale
                total = sum(t for _, t in members)
                for w, t in members:
                    w.encoder_seconds += dt * t / total
        check_finite = getattr(self.encode_tiles, "check_finite", None)
        if check_finite is not None:
            check_finite()


def _union_seconds(intervals: List[Tuple[float, float]]) -> float:
    total, end = 0.0, None
    for a, b in sorted(intervals):
        if end is None or a > end:
            total += b - a
            end = b
        elif b > end:
            total += b - end
            end = b
    return total


def _lanes_of(walks: List[_Traversal]) -> List[List[int]]:
    """Walks split into two lanes: those with the most blocks (the
    traversal's critical chain of calls) and the rest; one lane when every
    walk has the same length. On a 9B-class layer (down_proj 768 blocks,
    the other six 256) this measured 1.22 s against 1.30 s for one lane,
    and against 1.24-1.30 s for splits that move the smaller projections
    into the first lane."""
    longest = max(len(w.blocks) for w in walks)
    lanes = [[i for i, w in enumerate(walks) if len(w.blocks) == longest],
             [i for i, w in enumerate(walks) if len(w.blocks) < longest]]
    return [lane for lane in lanes if lane]


def _run_lockstep(walks: List[_Traversal], encode_tiles: TileEncoder,
                  synchronize: Optional[Callable[[], None]], time_calls: bool = True) -> None:
    """Every walk's blocks through the encoder, several walks per call as
    :func:`lockstep_schedule` assigns them.

    On a GPU, when the walks differ in length and the encoder can ``fork``
    a second adapter, the walks run as two lanes (:func:`_lanes_of`) on two
    streams, their calls queued alternately in proportion to their counts:
    one lane's latency-bound tracebacks and small launches then overlap the
    other's forward passes. Every walk's blocks still go through the
    encoder in order, so each result is unchanged. A walk's
    ``encoder_seconds`` is its tile share of each call's duration, the
    durations scaled so that all calls together count the time during which
    any was running; on a GPU without ``synchronize`` it is measured only
    with ``time_calls`` (HIP events around every call) and stays 0
    otherwise."""
    groups = _lanes_of(walks)
    concurrent = (len(groups) > 1 and walks[0].on_gpu and synchronize is None
                  and callable(getattr(encode_tiles, "fork", None)))
    if not concurrent:
        lane = _Lane(walks, encode_tiles, synchronize, time_calls=time_calls)
        while lane.done < len(lane.steps):
            lane.issue()
        lane.finish()
        return
    device = walks[0].weight.device
    origin = torch.cuda.current_stream(device)
    encoders = [encode_tiles] + [encode_tiles.fork() for _ in groups[1:]]
    # Tracebacks by per-row tree loads: the streamed kernel reads whole rows,
    # bandwidth the other lane's forward passes need (9B-class layer: 1.20 s
    # against 1.23-1.26 s). Each adapter carries its own choice, so nothing
    # process-wide changes and other threads' encodes are unaffected.
    previous_policy = getattr(encode_tiles, "traceback_policy", None)
    for enc in encoders:
        enc.traceback_policy = "rows"
    # The first lane stays on the caller's stream: two pool streams can share
    # one hardware queue, which would serialise the lanes again.
    ref = torch.cuda.Event(enable_timing=True)
    ref.record(origin)
    lanes = []
    try:
        for g, (members, enc) in enumerate(zip(groups, encoders)):
            stream = origin if g == 0 else torch.cuda.Stream(device=device)
            if g:
                stream.wait_stream(origin)
            with torch.cuda.stream(stream):
                lanes.append(_Lane([walks[i] for i in members], enc, None, stream,
                                   time_calls=time_calls))
        while True:
            open_lanes = [ln for ln in lanes if ln.done < len(ln.steps)]
            if not open_lanes:
                break
            lane = min(open_lanes, key=lambda ln: (ln.done + 1) / len(ln.steps))
            with torch.cuda.stream(lane.stream):
                lane.issue()
        for lane in lanes[1:]:
            origin.wait_stream(lane.stream)
        # Calls of different lanes overlap: their durations are scaled so
        # that together they add up to the time any encoder call was running.
        for lane in lanes:
            if lane.pending:
                lane.pending[-1][0][1].synchronize()
        spans = [iv for lane in lanes for iv in lane.intervals(ref)]
        busy = sum(b - a for a, b in spans)
        scale = _union_seconds(spans) / busy if busy > 0 else 1.0
        for lane in lanes:
            lane.finish(scale)
    finally:
        for lane in lanes[1:]:
            origin.wait_stream(lane.stream)
        encode_tiles.traceback_policy = previous_policy
        for enc in encoders[1:]:
            enc.encoder.arena.release()


def ldlq(weight: torch.Tensor, L: torch.Tensor, encode_tiles: TileEncoder,
         buf_size_k: int = DEFAULT_BUF_SIZE_K,
         synchronize: Callable[[], None] = None, time_calls: bool = True) -> LDLQResult:
    """Bottom-up one-sided LDLQ (ldlq.py:163-309). ``weight`` (k, n) float32
    in the transformed basis and ``L`` (k, k) from :func:`block_ldl` are not
    modified. ``encode_tiles`` maps (tiles_n, 256) tensor-core-order tiles to
    (reconstruction, int16 states).

    Bottom-up: spans of ``buf_size_k`` rows from the last, 16-row blocks
    inside a span from the last. A block's rows get the compensation of the
    rows already quantised below it in the span (``addmm`` against the
    strictly lower slice of L) plus the span-level feedback ``prod_cache``;
    after a span its residual is propagated into ``prod_cache``.

    ``encoder_seconds`` is the encoder's share: on a CUDA weight, with
    ``time_calls``, the sum of HIP-event intervals around each call on the
    current stream, read once after the traversal, so nothing in the loop
    waits for the device (0 without ``time_calls``: the events cost the
    stream about 5 us per call); with ``synchronize`` given, host wall time
    between two ``synchronize()`` calls around each call instead. An encoder exposing ``check_finite``
    (the HIP adapter) is asked once at the end to raise on NaN inputs."""
    walk = _Traversal(weight, L, buf_size_k)
    _run_lockstep([walk], encode_tiles, synchronize, time_calls)
    return walk.result()


def ldlq_lockstep(problems: Sequence[Tuple[torch.Tensor, torch.Tensor]],
                  encode_tiles: TileEncoder, buf_size_k: int = DEFAULT_BUF_SIZE_K,
                  synchronize: Callable[[], None] = None,
                  time_calls: bool = True) -> List[LDLQResult]:
    """:func:`ldlq` on several independent (weight, L) problems at once:
    each encoder call carries the next block of several problems, as
    :func:`lockstep_schedule` balances them (as many calls as the longest
    problem has blocks, each near the mean size), so a launch holds ~1000
    tiles instead of one projection's 64-768. Each result equals its own
    :func:`ldlq` run (tiles are encoded independently of their batch);
    ``encoder_seconds`` splits each call's time by the problems' tile
    counts."""
    if not problems:
        return []
    walks = [_Traversal(w, L, buf_size_k) for w, L in problems]
    devices = {w.weight.device for w in walks}
    if len(devices) != 1:
        raise ValueError(f"all problems must be on one device, got {sorted(map(str, devices))}")
    _run_lockstep(walks, encode_tiles, synchronize, time_calls)
    return [w.result() for w in walks]
