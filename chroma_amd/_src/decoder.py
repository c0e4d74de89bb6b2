"""KV-cached generation over a prefill/decode program pair.

Behaviour follows the reference ``Decoder`` (chroma/_src/decoder.py:44-152): programs exported by
``export_cached`` take (tokens, positions, K cache, V cache, full mask, window mask, logit row) and
return (logits, new K rows, new V rows); the cache is a rolling host buffer indexed by
``position % context``; masks are 0 where a cached or new key is causal and inside the window, -inf
elsewhere; one remaining token runs the decode graph, longer inputs run prefill in chunks; the cache
commits only after the native call returned, so an interrupted ``append`` leaves the last committed
state in place.

When both programs are hip programs the cache stays on the device (an extension: the reference keeps
it on the host and uploads all of it every step, decoder.py:68-76). Each program's own input staging
regions for the K and V caches hold a device copy; ``owner`` names the program whose copy is the
committed cache. A step uploads only tokens, positions, masks and the logit row, leaves the new K/V
rows in the program's output staging, and commits by copying those rows into the owner's cache rows
on the device; switching between prefill and decode first copies the committed cache across. The
device copy and the state update form one critical section that defers SIGINT, so an interrupt lands
either before the commit (state and device cache untouched) or after it.
"""

from __future__ import annotations

import _signal
import contextlib
import functools
import os
import shutil
import signal
import tempfile
import threading
from dataclasses import dataclass
from pathlib import Path
from typing import Any, Iterator, List, Optional, Sequence, Tuple

import numpy as np

from chroma_amd._src import host
from chroma_amd._src.dtypes import BFLOAT16, numpy_dtype
from chroma_amd._src.program import NativeModel, Program

SELECT_MAX_K = 1024  # largest k the runtime's row selection takes (chroma_hip_rows_topk)


@dataclass(frozen=True)
class CacheState:
    keys: Optional[np.ndarray]  # host cache (None when the cache lives on the device)
    values: Optional[np.ndarray]
    slots: np.ndarray  # absolute position held by each cache row, or -1
    position: int
    owner: Optional[int] = None  # device mode: the program whose staging holds the committed cache


@contextlib.contextmanager
def _interrupts_deferred() -> Iterator[None]:
    """Hold SIGINT until the block ends. Only the main thread receives it, and only a handler installed
    from Python can be put back afterwards; otherwise (a profiler's or embedder's native handler) the
    block runs as it is. The handlers are swapped through the C-level ``_signal`` module: ``signal.signal``
    converts handlers to and from enums, which cost 9 us of every decode step against 0.6 us."""
    previous = _signal.getsignal(_signal.SIGINT)
    if threading.current_thread() is not threading.main_thread() or previous is None:
        yield
        return
    pending: List[int] = []
    _signal.signal(_signal.SIGINT, lambda number, frame: pending.append(number))
    try:
        yield
    finally:
        _signal.signal(_signal.SIGINT, previous)
        if pending:
            os.kill(os.getpid(), signal.SIGINT)


def _staging_mirror(model: Program) -> List[Optional[np.ndarray]]:
    """The decoder's host input arrays (all but the caches, inputs 2 and 3) for a hip program: page-locked
    and placed at the same distances from each other as the program's input staging regions, one block
    per run of inputs adjacent in the staging (the caches end a run; a step's small inputs, staged ahead of
    the caches, form one run and go up as one copy)."""
    native = model.native
    specs = model.inputs
    arrays: List[Optional[np.ndarray]] = [None] * len(specs)
    staged = sorted(range(len(specs)), key=native.input_pointer)
    runs: List[List[int]] = [[]]
    for i in staged:
        if i in (2, 3):
            runs.append([])
        else:
            runs[-1].append(i)
    for run in (run for run in runs if run):
        start = native.input_pointer(run[0])
        sizes = [int(np.prod(specs[i]["shape"])) * numpy_dtype(specs[i]["dtype"]).itemsize for i in run]
        span = native.input_pointer(run[-1]) - start + sizes[-1]
        block = host.empty((span,), np.uint8)
        for i, size in zip(run, sizes):
            at = native.input_pointer(i) - start
            arrays[i] = block[at : at + size].view(numpy_dtype(specs[i]["dtype"])).reshape(specs[i]["shape"])
    return arrays


def _fill_row(mask: np.ndarray, allowed: np.ndarray) -> None:
    """A one-step mask [1, context + 1]: 0 where ``allowed`` over the cached keys, and 0 for the new key.
    Written through the bit patterns: (not allowed) x the -inf pattern, one ufunc per row."""
    if mask.dtype == np.float32:
        bits = mask.view(np.uint32)[0]
        np.multiply(~allowed, np.uint32(0xFF800000), out=bits[:-1])
    else:
        bits = mask.view(np.uint16)[0]
        np.multiply(~allowed, np.uint16(0xFF80), out=bits[:-1])
    bits[-1] = 0


def _fill_mask(mask: np.ndarray, allowed: np.ndarray) -> None:
    """0 where ``allowed``, -inf elsewhere (bfloat16 masks are written through their bit patterns)."""
    if mask.dtype == np.float32:
        mask.fill(-np.inf)
        mask[allowed] = 0
    else:
        bits = mask.view(np.uint16)
        bits.fill(0xFF80)
        bits[allowed] = 0


@functools.lru_cache(maxsize=8)
def _band(steps: int, window: int, bits: str) -> np.ndarray:
    """Mask bits over the new keys of a multi-step call: key c (time position + c) is blocked for query t
    when c > t or c <= t - window, whatever the position. Read-only, shared by every call of this shape."""
    c = np.arange(steps)
    blocked = (c[None, :] > c[:, None]) | (c[None, :] <= c[:, None] - window)
    dtype = np.dtype(bits)
    out = np.multiply(blocked, dtype.type(0xFF800000 if dtype.itemsize == 4 else 0xFF80), dtype=dtype)
    out.setflags(write=False)
    return out


def _fill_masks(masks: Sequence[Tuple[np.ndarray, int]], key_times: np.ndarray, valid: np.ndarray, times: np.ndarray) -> None:
    """Multi-step masks [steps, keys], one per (mask, window): 0 where key j is valid, not after query t
    (key_times[j] <= times[t]) and inside the window (key_times[j] > times[t] - window), -inf elsewhere.
    The keys are the cached ones followed by the new ones, whose times are ``times`` (always valid): that
    block is a band fixed by (steps, window) and copied from a cache. Cached keys are all blocked when none
    is valid (a fresh prefill); otherwise invalid keys take the largest time, so "after the query" covers
    them, and the block is the blocked indicator times the -inf bit pattern (two comparisons and a
    multiply, no boolean index assignment)."""
    steps = len(times)
    past = len(key_times) - steps
    valid_past = valid[:past]
    any_valid = bool(valid_past.any())
    if any_valid:
        kt = np.where(valid_past, key_times[:past], np.iinfo(np.int64).max)
        late = kt[None, :] > times[:, None]
        blocked = np.empty_like(late)
    for mask, window in masks:
        bits = np.uint32 if mask.dtype == np.float32 else np.uint16
        view = mask.view(bits)
        neg = bits(0xFF800000 if bits is np.uint32 else 0xFF80)
        if any_valid:
            np.less_equal(kt[None, :], (times - window)[:, None], out=blocked)
            np.logical_or(blocked, late, out=blocked)
            np.multiply(blocked, neg, out=view[:, :past])
        else:
            view[:, :past] = neg
        view[:, past:] = _band(steps, window, np.dtype(bits).str)


def _validate(prefill: Program, decode: Program, extra_outputs: bool = False) -> Tuple[dict, dict]:
    for name, model in (("prefill", prefill), ("decode", decode)):
        if len(model.inputs) != 7 or len(model.outputs) != 3 and not (extra_outputs and len(model.outputs) > 3):
            raise ValueError(f"Decoder {name} wants seven inputs and three outputs, not {len(model.inputs)} and {len(model.outputs)}")
    if len(prefill.outputs) != len(decode.outputs):
        raise ValueError("Decoder prefill and decode were not exported as a pair")
    cache, logits = decode.inputs[2], decode.outputs[0]
    steps = prefill.inputs[0]["shape"][0]
    if (
        decode.inputs[0]["shape"] != [1]
        or prefill.inputs[2]["shape"] != cache["shape"]
        or prefill.outputs[0]["shape"] != logits["shape"]
        or not 1 <= steps <= cache["shape"][1]
    ):
        raise ValueError("Decoder prefill and decode were not exported as a pair")
    return cache, logits


def _select_host(row: np.ndarray, k: int, ids: Optional[np.ndarray]) -> Tuple[np.ndarray, np.ndarray]:
    """The top-k rule of ``Decoder.append_top`` on a downloaded logits row: NaN first, then values
    descending, ties to the lower id (a stable sort)."""
    candidates = row if ids is None else row[ids]
    wide = candidates.astype(np.float32)
    nan = np.isnan(wide)
    # lexsort is stable and sorts by its last key first: NaN before any number (+inf included), then
    # larger values first, ties in id order.
    order = np.lexsort((np.where(nan, 0, -wide), ~nan))[:k]
    return candidates[order].copy(), (order if ids is None else ids[order]).astype(np.int64)


class _TopK:
    """Selection program of ``append_top``: top-k of the logits row."""

    def __new__(cls, k: int):
        import torch

        class TopK(torch.nn.Module):
            def forward(self, logits):
                return torch.topk(logits, k, dim=-1)

        return TopK()


class _GatheredTopK:
    """Selection program of ``append_top`` with ``allowed``: top-k among the gathered candidate ids."""

    def __new__(cls, k: int):
        import torch

        class GatheredTopK(torch.nn.Module):
            def forward(self, logits, ids):
                return torch.topk(logits.reshape(-1)[ids].reshape(1, -1), k, dim=-1)

        return GatheredTopK()


class Decoder:
    def __init__(self, prefill: Program, decode: Program, *, sliding_window: int = 0, extra_outputs: bool = False) -> None:
        """``extra_outputs`` (an addition to the reference API) accepts programs that return more than the
        three outputs (logits, new K rows, new V rows), such as ``export_cached(..., routing=True)``
        probes; after each ``append`` the ``extras`` property holds, per program run, the first position
        it consumed, its token count and copies of its extra outputs."""
        if sliding_window < 0:
            raise ValueError(f"sliding_window must be nonnegative, got {sliding_window}")
        cache, logits = _validate(prefill, decode, extra_outputs)
        self._models = (prefill, decode)
        self._shape = tuple(cache["shape"])
        self._cache_dtype = numpy_dtype(cache["dtype"])
        self._logit_dtype = numpy_dtype(logits["dtype"])
        self.context = self._shape[1]
        self.vocab_size = logits["shape"][1]
        self.device = decode.device
        self._window = min(sliding_window or self.context, self.context)
        self._on_device = all(isinstance(model, Program) for model in self._models) and prefill.device == decode.device
        # Per program: the seven input arrays (the caches are bound at commit time, or stay on the
        # device) and the host arrays for the new K/V rows (device mode leaves those on the device).
        # (With hip programs the host arrays are page-locked, so their copies go straight over the link, and
        # laid out like the program's input staging, so each run of them goes up as one copy.)
        empty = host.empty if self._on_device else np.empty
        self._empty_array = empty
        self._buffers: List[Tuple[List[Optional[np.ndarray]], List[Optional[np.ndarray]], List[np.ndarray]]] = [
            (
                _staging_mirror(model) if self._on_device and isinstance(model.native, NativeModel)
                else [None if i in (2, 3) else empty(spec["shape"], numpy_dtype(spec["dtype"])) for i, spec in enumerate(model.inputs)],
                [None if self._on_device else np.empty(spec["shape"], dtype=numpy_dtype(spec["dtype"])) for spec in model.outputs[1:3]],
                [empty(spec["shape"], numpy_dtype(spec["dtype"])) for spec in model.outputs[3:]],
            )
            for model in self._models
        ]
        # Multi-step hip programs build their masks on the device (NativeModel.decoder_masks).
        self._device_masks = [self._on_device and isinstance(model.native, NativeModel) and model.inputs[0]["shape"][0] > 1
                              for model in self._models]
        self._extras: List[Tuple[int, int, List[np.ndarray]]] = []
        self._row_bytes = int(np.prod(self._shape[2:])) * self._cache_dtype.itemsize
        self._selectors: dict = {}  # (k, gathered ids or None) -> top-k selection program (hip pairs)
        self._selector_dir: Optional[str] = None
        self._lock = threading.RLock()  # re-entered by append_top around its step and selection
        self._closed = False
        self._commit(self._empty())

    def _empty(self) -> CacheState:
        slots = np.full(self.context, -1, dtype=np.int64)
        if self._on_device:
            return CacheState(None, None, slots, 0)
        keys = np.zeros(self._shape, dtype=self._cache_dtype)
        return CacheState(keys, np.zeros_like(keys), slots, 0)

    def _commit(self, state: CacheState) -> None:
        self._state = state
        if not self._on_device:
            for args, _, _ in self._buffers:
                args[2], args[3] = state.keys, state.values

    # ---------------------------------------------------------------------------- device-resident cache
    def _device_cache(self, which: int, args: List[Any]) -> None:
        """Make program ``which``'s device copy of the cache the committed cache: zero a fresh cache (on the
        device for hip programs, else by uploading zeros), copy from the owner's staging when another
        program owns it, or leave it (args None)."""
        owner = self._state.owner
        if owner is None:
            native = self._models[which].native
            if isinstance(native, NativeModel):
                native.clear_input(2)
                native.clear_input(3)
                args[2] = args[3] = None
            else:
                zeros = np.zeros(self._shape, dtype=self._cache_dtype)
                args[2], args[3] = zeros, zeros
            return
        args[2] = args[3] = None
        if owner != which:
            target, source = self._models[which].native, self._models[owner].native
            source.synchronize()  # its queued commits have landed
            size = int(np.prod(self._shape)) * self._cache_dtype.itemsize
            for index in (2, 3):
                target.copy_2d(target.input_pointer(index), size, source.input_pointer(index), size, size, 1)

    def _device_commit(self, which: int, start: int, count: int, steps: int) -> None:
        """Copy the first ``count`` new K/V rows of program ``which`` (its outputs 1 and 2, [layers, steps,
        ...]) into its cache inputs (2 and 3, [layers, context, ...]) at rows (start + i) % context."""
        program = self._models[which].native
        row, layers = self._row_bytes, self._shape[0]
        first = start % self.context
        head = min(count, self.context - first)
        # Queued on the program's stream, all in one launch: its next run (or a synchronize before another
        # program copies the cache) comes after them.
        rects = []
        for output, cache in ((1, 2), (2, 3)):
            src, dst = program.output_pointer(output), program.input_pointer(cache)
            rects.append((dst + first * row, self.context * row, src, steps * row, head * row, layers))
            if count > head:
                rects.append((dst, self.context * row, src + head * row, steps * row, (count - head) * row, layers))
        program.copy_2d_batch(rects)

    @property
    def position(self) -> int:
        return self._state.position

    @property
    def extras(self) -> List[Tuple[int, int, List[np.ndarray]]]:
        """The last ``append``'s extra outputs: (first position, tokens, arrays) per program run."""
        return list(self._extras)

    @property
    def stats(self) -> dict:
        return {
            "cache_bytes": 2 * int(np.prod(self._shape)) * self._cache_dtype.itemsize,
            "cache_on_device": self._on_device,
            "prefill": self._models[0].stats,
            "decode": self._models[1].stats,
        }

    def reset(self) -> None:
        with self._lock:
            if self._closed:
                raise RuntimeError("Decoder is closed")
            self._commit(self._empty())

    def append(self, tokens: Any) -> np.ndarray:
        """Consume new token ids and return the logits [1, vocab] after the last one."""
        logits, _, _ = self._consume(tokens, keep_logits=False)
        return logits

    def append_top(self, tokens: Any, k: int = 1, *, allowed: Any = None) -> Tuple[np.ndarray, np.ndarray]:
        """Consume new token ids like ``append`` and return the ``k`` largest logits after the last one
        with their token ids, largest first: NaN outranks every number and ties go to the lower id (the
        reference GPU backend's top-k rule). ``allowed`` (token ids) restricts the choice to those ids.

        With hip programs the logits never leave the device: the runtime's row selection runs on the step's
        own stream right after it, under the step's one synchronization, and only the ``k`` values and ids
        come back instead of the vocabulary row (k up to 1024). With ``allowed``, a small selection
        program (a gather of the allowed ids, then the top-k kernel) reads the step's logits by a
        device-to-device copy instead. Other programs select on the host by the same rule. (An addition to
        the reference API: its chat script samples from the downloaded row, scripts/chat.py:82-98.)"""
        if not isinstance(k, (int, np.integer)) or k < 1:
            raise ValueError(f"k must be a positive integer, got {k!r}")
        ids = None
        if allowed is not None:
            ids = np.unique(np.asarray(allowed))
            if ids.ndim != 1 or not np.issubdtype(ids.dtype, np.integer):
                raise TypeError("allowed must be a 1-D sequence of integer token ids")
            if len(ids) and (ids[0] < 0 or ids[-1] >= self.vocab_size):
                raise IndexError(f"allowed token ids must lie in [0, {self.vocab_size})")
            ids = ids.astype(np.int64)
        if k > (len(ids) if ids is not None else self.vocab_size):
            raise ValueError(f"k = {k} exceeds the number of candidate tokens")
        device = self._on_device and isinstance(self._models[1].native, NativeModel)
        with self._lock:  # the step's device logits stay this step's until the selection has read them
            if device and ids is None and k <= SELECT_MAX_K:
                _, _, (values, picks) = self._consume(tokens, keep_logits=True, top=int(k))
                return values[0].copy(), picks[0].copy()
            logits, which, _ = self._consume(tokens, keep_logits=device)
            if not device:
                return _select_host(logits[0], int(k), ids)
            selector = self._selector(int(k), None if ids is None else len(ids))
            native = selector.native
            row = self.vocab_size * self._logit_dtype.itemsize
            # queued on the selection program's stream, so its run comes after the copy without a wait here
            # (the step's run has finished; the next step cannot start before this call returns)
            native.copy_2d(native.input_pointer(0), row, self._models[which].native.output_pointer(0), row, row, 1, queued=True)
            values = host.empty((1, int(k)), self._logit_dtype)
            picks = host.empty((1, int(k)), np.int64)
            if ids is None:
                selector.run_resident([None], [values, picks])
                return values[0].copy(), picks[0].copy()
            selector.run_resident([None, ids], [values, picks])
            return values[0].copy(), ids[picks[0]]

    def greedy(self, tokens: Any, *, allowed: Any = None) -> int:
        """Consume new token ids and return the id of the largest logit after the last one (``append_top``
        with k = 1)."""
        return int(self.append_top(tokens, 1, allowed=allowed)[1][0])

    def _selector(self, k: int, candidates: Optional[int]) -> Program:
        """The hip program selecting the top ``k`` of a logits row (of ``candidates`` gathered ids), compiled
        on first use next to the decoder's programs and kept until ``close``."""
        key = (k, candidates)
        program = self._selectors.get(key)
        if program is None:
            import torch

            from chroma_amd._src.compiler import compile_for_backend

            dtype = torch.bfloat16 if self._logit_dtype == BFLOAT16 else getattr(torch, np.dtype(self._logit_dtype).name)
            logits = torch.zeros(1, self.vocab_size, dtype=dtype)
            if candidates is None:
                example, module = (logits,), _TopK(k)
            else:
                example, module = (logits, torch.zeros(candidates, dtype=torch.int64)), _GatheredTopK(k)
            if self._selector_dir is None:
                self._selector_dir = tempfile.mkdtemp(prefix="chroma-select-")
            target = Path(self._selector_dir) / f"top{k}-{candidates or 'all'}"
            program = compile_for_backend(torch.export.export(module, example), target, backend="hip")
            self._selectors[key] = program
        return program

    def _consume(self, tokens: Any, *, keep_logits: bool, top: Optional[int] = None) -> Tuple[Optional[np.ndarray], int, Any]:
        """Run the steps for ``tokens``; return the last step's logits (None when ``keep_logits`` leaves
        them in the device output of the program that ran it), that program's index, and, when ``top`` is
        given (device mode), the (values, ids) of the last step's ``top`` largest logits selected on the
        device after it."""
        ids = np.asarray(tokens)
        if ids.ndim != 1 or not len(ids):
            raise ValueError(f"append wants a nonempty 1-D sequence of token IDs, got shape {ids.shape}")
        if not np.issubdtype(ids.dtype, np.integer):
            raise TypeError(f"Token IDs must be integers, got {ids.dtype}")
        ids = ids.astype(np.int64)
        with self._lock:
            if self._closed:
                raise RuntimeError("Decoder is closed")
            offset = 0
            logits = None
            selection = None
            which = 1
            self._extras = []
            while offset < len(ids):
                remaining = len(ids) - offset
                which = 1 if remaining == 1 else 0
                args, updates, extras = self._buffers[which]
                steps = len(args[0])
                count = min(steps, remaining)
                state = self._state
                times = state.position + np.arange(steps, dtype=np.int64)
                token_ids, positions, _, _, full_mask, window_mask, logit_index = args
                token_ids.fill(0)
                token_ids[:count] = ids[offset : offset + count]
                positions[:] = times
                if steps == 1:
                    # One new key at the current position: every committed key is older, so the causal
                    # test reduces to validity (slot >= 0) and each window test to one comparison; the two
                    # combine into slot > max(position - window, -1). Equal windows share one row.
                    _fill_row(full_mask, state.slots > max(state.position - self.context, -1))
                    if self._window == self.context:
                        np.copyto(window_mask, full_mask)
                    else:
                        _fill_row(window_mask, state.slots > max(state.position - self._window, -1))
                elif self._device_masks[which]:
                    # Built on the device into the mask inputs' staging (the next run is given None for them):
                    # two [steps, context + steps] masks never cross the host link.
                    self._models[which].native.decoder_masks(state.slots, state.position, steps, self._window, 4, 5)
                else:
                    _fill_masks(((full_mask, self.context), (window_mask, self._window)), np.concatenate((state.slots, times)),
                                np.concatenate((state.slots >= 0, np.ones(steps, dtype=bool))), times)
                logit_index[0] = count - 1
                logits = None if keep_logits else self._empty_array((1, self.vocab_size), self._logit_dtype)
                rows = times[:count] % self.context
                slots = state.slots.copy()
                slots[rows] = times[:count]
                if self._on_device:
                    self._device_cache(which, args)
                    inputs = args
                    if self._device_masks[which]:
                        inputs = list(args)
                        inputs[4] = inputs[5] = None  # the masks built on the device above
                    if top is not None and offset + count == len(ids):
                        selection = self._models[which].run_top_resident(inputs, [logits, *updates, *extras], 0, top)
                    else:
                        self._models[which].run_resident(inputs, [logits, *updates, *extras])
                    with _interrupts_deferred():
                        self._device_commit(which, state.position, count, steps)
                        self._commit(CacheState(None, None, slots, state.position + count, which))
                else:
                    self._models[which](*args, out=[logits, *updates, *extras])
                    keys, values = state.keys.copy(), state.values.copy()
                    keys[:, rows] = updates[0][:, :count]
                    values[:, rows] = updates[1][:, :count]
                    self._commit(CacheState(keys, values, slots, state.position + count))
                if extras:
                    self._extras.append((state.position, count, [array.copy() for array in extras]))
                offset += count
            return logits, which, selection

    def close(self) -> None:
        with self._lock:
            for model in self._models:
                model.close()
            for program in self._selectors.values():
                program.close()
            self._selectors.clear()
            if self._selector_dir is not None:
                shutil.rmtree(self._selector_dir, ignore_errors=True)
                self._selector_dir = None
            self._closed = True
            self._buffers.clear()

    def __enter__(self) -> "Decoder":
        return self

    def __exit__(self, *exc: Any) -> None:
        self.close()
