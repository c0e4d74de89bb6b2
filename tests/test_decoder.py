"""The KV-cached ``Decoder`` on the CPU (mirrors the reference's tests/test_decoder.py:42-147).

The program pair is the oracle (the CPU restatement of Chroma's CPU backend), so these run without a GPU:
construction checks with mock programs, prefill / decode / wrap-around / reset against an eager causal
forward, rejected token ids, and an interrupt after the native call. The device-resident cache path that
hip programs take is exercised against a stand-in device (host memory addressed like device memory, the
oracle computing), which must reproduce the host-cache decoder step for step.
"""

from __future__ import annotations

import copy
import dataclasses
import os
import signal
import threading
from typing import Any, List, Optional
from unittest.mock import Mock, patch

import numpy as np
import pytest
import torch

from chroma_amd import Decoder, Program
from chroma_amd._src.dtypes import BFLOAT16
from chroma_amd._src.decoder import _interrupts_deferred
from chroma_amd.models.cached import export_cached
from chroma_amd.models.variants import dev
from oracle import compile_cpu
from tests.helpers import random_transformer


def small_model(head_dim: int = 8):
    config = dataclasses.replace(
        dev,
        num_hidden_layers=2,
        hidden_size=16,
        intermediate_size=16,
        vocab_size=31,
        num_experts=4,
        experts_per_token=2,
        num_attention_heads=4,
        num_key_value_heads=2,
        head_dim=head_dim,
        sliding_window=3,
        initial_context_length=4096,
        rope_scaling_factor=32.0 if head_dim == 64 else 1.0,
    )
    return random_transformer(config, seed=5, std=0.03)


def mock_program(steps: int, capacity: int = 7, vocabulary: int = 5) -> Program:
    cache = [2, capacity, 1, 4]
    inputs = [([steps], "int64"), ([steps], "float32"), (cache, "float32"), (cache, "float32"),
              ([steps, capacity + steps], "float32"), ([steps, capacity + steps], "float32"), ([1], "int64")]
    outputs = [([1, vocabulary], "float32"), ([2, steps, 1, 4], "float32"), ([2, steps, 1, 4], "float32")]
    return Mock(
        spec=Program,
        device="CPU",
        inputs=[{"name": str(i), "shape": shape, "dtype": dtype} for i, (shape, dtype) in enumerate(inputs)],
        outputs=[{"name": str(i), "shape": shape, "dtype": dtype} for i, (shape, dtype) in enumerate(outputs)],
    )


def test_incompatible_program_pairs_fail_at_construction():
    with Decoder(mock_program(3), mock_program(1)) as decoder:
        assert (decoder.context, decoder.vocab_size) == (7, 5)
    pairs = ((mock_program(3, capacity=4), mock_program(1)), (mock_program(3, vocabulary=3), mock_program(1)), (mock_program(3), mock_program(2)))
    for prefill, decode in pairs:
        with pytest.raises(ValueError, match="Decoder"):
            Decoder(prefill, decode)
    broken = mock_program(1)
    broken.inputs = []
    with pytest.raises(ValueError, match="seven inputs"):
        Decoder(mock_program(3), broken)


def test_reject_invalid_sliding_window():
    program = Mock(spec=Program)
    for window in (-1, -7):
        with pytest.raises(ValueError, match="sliding_window"):
            Decoder(program, program, sliding_window=window)


@pytest.fixture(scope="module")
def oracle_pairs(tmp_path_factory):
    """Oracle prefill/decode programs (context 7) and the eager causal logits, for head_dim 8 and 64."""
    context = 7
    pairs = {}
    for head_dim in (8, 64):
        eager = small_model(head_dim)
        reference = copy.deepcopy(eager)
        for block in reference.block:
            block.attn.sliding_window = min(block.attn.sliding_window or context, context)
        tokens = (torch.arange(23) * 7 + 3) % 31
        with torch.no_grad():
            expected = reference(tokens).numpy()
        root = tmp_path_factory.mktemp(f"decoder{head_dim}")
        graphs = [export_cached(eager, context, steps) for steps in (context, 1)]
        pairs[head_dim] = (graphs, [compile_cpu(g, root / f"p{i}") for i, g in enumerate(graphs)], tokens.numpy(), expected)
    return pairs


@pytest.mark.parametrize("head_dim", [8, 64])
def test_prefill_decode_wrap_and_reset_match_causal_reference(oracle_pairs, head_dim):
    _, (prefill, decode), tokens, expected = oracle_pairs[head_dim]
    cached = Decoder(prefill, decode, sliding_window=3)
    assert not cached.stats["cache_on_device"]
    position = 0
    for size in (3, 1, 5, 7, 1, 6):
        logits = cached.append(tokens[position : position + size])
        position += size
        np.testing.assert_allclose(logits, expected[position - 1 : position], rtol=2e-5, atol=2e-6)
        assert cached.position == position
    preserved = logits.copy()
    cached.reset()
    np.testing.assert_allclose(cached.append(tokens), expected[-1:], rtol=2e-5, atol=2e-6)
    cached.reset()
    assert cached.position == 0
    np.testing.assert_allclose(cached.append(tokens[:3]), expected[2:3], rtol=2e-5, atol=2e-6)
    np.testing.assert_array_equal(logits, preserved)
    for invalid in ([-1], [31], [2**40]):
        with pytest.raises(IndexError):
            cached.append(invalid)
        assert cached.position == 3
    with pytest.raises(TypeError):
        cached.append([1.5])
    with pytest.raises(ValueError):
        cached.append([])
    before = cached._state
    step = cached._models[1]

    def interrupted(*args, out=None):
        step(*args, out=out)
        raise KeyboardInterrupt

    with patch.object(cached, "_models", (cached._models[0], interrupted)), pytest.raises(KeyboardInterrupt):
        cached.append([int(tokens[3])])
    assert cached._state is before
    np.testing.assert_allclose(cached.append([int(tokens[3])]), expected[3:4], rtol=2e-5, atol=2e-6)


# ----------------------------------------------------------------------------------- device-resident cache
class FakeDevice:
    """Byte-addressed stand-in for device memory: addresses are offsets into one host buffer (from 4096,
    so no address is 0)."""

    def __init__(self, size: int) -> None:
        self.memory = np.zeros(size, dtype=np.uint8)
        self.top = 4096

    def allocate(self, nbytes: int) -> int:
        address = self.top
        self.top += -(-nbytes // 256) * 256
        assert self.top <= self.memory.size
        return address

    def view(self, address: int, spec: dict) -> np.ndarray:
        from chroma_amd._src.dtypes import numpy_dtype

        dtype = numpy_dtype(spec["dtype"])
        count = int(np.prod(spec["shape"]))
        return self.memory[address : address + count * dtype.itemsize].view(dtype).reshape(spec["shape"])


class FakeNative:
    """The device-resident surface of a hip program (run with None entries, staging pointers, copy_2d)
    over ``FakeDevice`` memory, computing with an oracle program."""

    def __init__(self, oracle, device: FakeDevice) -> None:
        self.oracle, self.device = oracle, device
        self.inputs = [device.allocate(int(np.prod(s["shape"])) * 8) for s in oracle.inputs]
        self.outputs = [device.allocate(int(np.prod(s["shape"])) * 8) for s in oracle.outputs]
        self.copies = 0
        self.pending: List[Any] = []

    def input_pointer(self, index: int) -> int:
        return self.inputs[index]

    def output_pointer(self, index: int) -> int:
        return self.outputs[index]

    def copy_2d(self, dst, dst_pitch, src, src_pitch, width, height, *, queued=False) -> None:
        # A queued copy happens only when this program's stream reaches it: at its next run, copy or
        # synchronize (so a reader on another program that skips ``synchronize`` sees stale rows).
        assert dst_pitch >= width and src_pitch >= width

        def copy():
            for row in range(height):
                self.device.memory[dst + row * dst_pitch : dst + row * dst_pitch + width] = self.device.memory[src + row * src_pitch : src + row * src_pitch + width]

        self.pending.append(copy)
        self.copies += 1
        if not queued:
            self.synchronize()

    def copy_2d_batch(self, rects) -> None:
        # one queued launch copying every rectangle, in order
        assert 1 <= len(rects) <= 4
        for rect in rects:
            self.copy_2d(*rect, queued=True)

    def synchronize(self) -> None:
        for copy in self.pending:
            copy()
        self.pending.clear()

    def run(self, inputs: List[Optional[np.ndarray]], outputs: List[Optional[np.ndarray]], *, resident: bool) -> None:
        self.synchronize()
        staged = [self.device.view(address, spec) for address, spec in zip(self.inputs, self.oracle.inputs)]
        for value, target in zip(inputs, staged):
            if value is not None:
                target[...] = value
        results = self.oracle(*staged)
        for value, address, spec in zip(results, self.outputs, self.oracle.outputs):
            self.device.view(address, spec)[...] = value
        for value, address, spec in zip(outputs, self.outputs, self.oracle.outputs):
            if value is not None:
                value[...] = self.device.view(address, spec)


class FakeDeviceProgram(Program):
    def __init__(self, oracle, device: FakeDevice) -> None:  # no artifact: state set directly
        self._lock = threading.Lock()
        self._model = FakeNative(oracle, device)
        self._inputs, self._outputs, self._stats, self._device = oracle.inputs, oracle.outputs, oracle.stats, "fake device"


@pytest.mark.parametrize("head_dim", [8, 64])
def test_device_resident_cache_matches_host_cache(oracle_pairs, head_dim):
    _, (prefill, decode), tokens, expected = oracle_pairs[head_dim]
    device = FakeDevice(1 << 22)
    fake = [FakeDeviceProgram(prefill, device), FakeDeviceProgram(decode, device)]
    resident, host = Decoder(*fake, sliding_window=3), Decoder(prefill, decode, sliding_window=3)
    assert resident.stats["cache_on_device"]
    position = 0
    for size in (3, 1, 1, 5, 7, 1, 4, 1):
        got, want = resident.append(tokens[position : position + size]), host.append(tokens[position : position + size])
        np.testing.assert_array_equal(got, want)
        position += size
        assert resident.position == host.position == position
        np.testing.assert_array_equal(resident._state.slots, host._state.slots)
        owner = fake[resident._state.owner].native
        owner.synchronize()  # the commit's copies are queued on the owner's stream
        for index, cache in ((2, host._state.keys), (3, host._state.values)):
            np.testing.assert_array_equal(device.view(owner.input_pointer(index), prefill.inputs[index]), cache)
    np.testing.assert_allclose(got, expected[position - 1 : position], rtol=2e-5, atol=2e-6)
    resident.reset()
    host.reset()
    np.testing.assert_array_equal(resident.append(tokens[:3]), host.append(tokens[:3]))
    with pytest.raises(IndexError):
        resident.append([31])
    assert resident.position == 3
    # An interrupt after the native call and before the commit leaves the committed state in place.
    before = resident._state
    run = fake[1].native.run

    def interrupted(inputs, outputs, *, resident):
        run(inputs, outputs, resident=resident)
        raise KeyboardInterrupt

    with patch.object(fake[1].native, "run", interrupted), pytest.raises(KeyboardInterrupt):
        resident.append([int(tokens[3])])
    assert resident._state is before
    np.testing.assert_array_equal(resident.append([int(tokens[3])]), host.append([int(tokens[3])]))


def test_interrupts_deferred_until_commit_ends():
    reached = []
    with pytest.raises(KeyboardInterrupt):
        with _interrupts_deferred():
            os.kill(os.getpid(), signal.SIGINT)
            reached.append("inside")
    assert reached == ["inside"]
    assert signal.getsignal(signal.SIGINT) is signal.default_int_handler


def test_one_step_masks_match_the_general_rule():
    """The single-token mask path (validity and one window comparison per cached key) writes the same
    float32 and bfloat16 masks as the general causal/window rule, over every cache state a decoder of
    context 7 passes through, before and after wrapping."""
    from chroma_amd._src.decoder import _fill_mask, _fill_row

    context = 7
    for position in range(40):
        slots = np.full(context, -1, dtype=np.int64)
        for t in range(max(0, position - context), position):
            slots[t % context] = t
        times = position + np.arange(1)
        key_times = np.concatenate((slots, times))
        valid = np.concatenate((slots >= 0, [True]))
        causal = valid[None] & (key_times[None] <= times[:, None])
        for window in range(1, context + 1):
            for dtype in (np.float32, np.uint16):
                general, fast = np.empty((1, context + 1), dtype), np.empty((1, context + 1), dtype)
                as_mask = (lambda m: m) if dtype == np.float32 else (lambda m: m.view(BFLOAT16))
                _fill_mask(as_mask(general), causal & (key_times[None] > times[:, None] - window))
                _fill_row(as_mask(fast), (slots >= 0) & (slots > position - window))
                np.testing.assert_array_equal(general.view(np.uint8), fast.view(np.uint8))


def test_top_k_selection_rule():
    """``append_top``'s rule: NaN first, values descending, ties to the lower id; ``allowed`` restricts the
    candidates and its ids come back, ties still to the lower id."""
    from chroma_amd._src.decoder import _select_host

    row = np.array([1.0, 3.0, np.nan, 3.0, -np.inf, 2.0, 3.0], dtype=np.float32)
    values, ids = _select_host(row, 4, None)
    np.testing.assert_array_equal(ids, [2, 1, 3, 6])
    np.testing.assert_array_equal(values[1:], [3.0, 3.0, 3.0])
    assert np.isnan(values[0])
    values, ids = _select_host(row, 3, np.array([0, 4, 5, 6]))
    np.testing.assert_array_equal(ids, [6, 5, 0])
    np.testing.assert_array_equal(values, [3.0, 2.0, 1.0])
    # NaN outranks +inf even when the +inf has the lower id; NaNs among themselves go by id
    row = np.array([np.inf, 1.0, np.nan, np.inf, np.nan], dtype=np.float32)
    values, ids = _select_host(row, 5, None)
    np.testing.assert_array_equal(ids, [2, 4, 0, 3, 1])
    np.testing.assert_array_equal(values[2:], [np.inf, np.inf, 1.0])


def test_append_top_on_host_programs_matches_logits(oracle_pairs):
    """Programs that are not hip programs select on the host: ``append_top`` / ``greedy`` agree with the
    logits ``append`` returns for the same tokens, and bad arguments are rejected."""
    from chroma_amd._src.decoder import _select_host

    _, (prefill, decode), tokens, _ = oracle_pairs[8]
    selecting, full = Decoder(prefill, decode, sliding_window=3), Decoder(prefill, decode, sliding_window=3)
    values, ids = selecting.append_top(tokens[:3], 4)
    want = _select_host(full.append(tokens[:3])[0], 4, None)
    np.testing.assert_array_equal(ids, want[1])
    np.testing.assert_array_equal(values, want[0])
    assert selecting.greedy([int(tokens[3])]) == int(_select_host(full.append([int(tokens[3])])[0], 1, None)[1][0])
    values, ids = selecting.append_top([int(tokens[4])], 2, allowed=[7, 3, 3, 20])
    want = _select_host(full.append([int(tokens[4])])[0], 2, np.array([3, 7, 20]))
    np.testing.assert_array_equal(ids, want[1])
    for bad, error in (({"k": 0}, ValueError), ({"k": 4, "allowed": [1, 2]}, ValueError), ({"allowed": [31]}, IndexError)):
        with pytest.raises(error):
            selecting.append_top([1], **bad)
    assert selecting.position == 5


def test_multi_step_masks_match_the_general_rule():
    """The multi-step mask writer (blocked indicator times the -inf bits) equals the general rule
    (valid, causal, inside the window -> 0; else -inf) in float32 and bfloat16, over random cache states
    with invalid, old, wrapped and new keys."""
    from chroma_amd._src.decoder import _fill_mask, _fill_masks

    rng = np.random.default_rng(3)
    for trial in range(40):
        context, steps = int(rng.integers(2, 12)), int(rng.integers(1, 9))
        position = int(rng.integers(0, 30))
        slots = np.where(rng.random(context) < 0.3, -1, rng.integers(0, max(position, 1), context)).astype(np.int64)
        times = position + np.arange(steps, dtype=np.int64)
        key_times = np.concatenate((slots, times))
        valid = np.concatenate((slots >= 0, np.ones(steps, dtype=bool)))
        causal = valid[None] & (key_times[None] <= times[:, None])
        for dtype in (np.float32, np.uint16):
            as_mask = (lambda m: m) if dtype == np.float32 else (lambda m: m.view(BFLOAT16))
            windows = (context, int(rng.integers(1, context + 1)))
            fast = [np.empty((steps, context + steps), dtype) for _ in windows]
            _fill_masks([(as_mask(m), w) for m, w in zip(fast, windows)], key_times, valid, times)
            for mask, window in zip(fast, windows):
                general = np.empty_like(mask)
                _fill_mask(as_mask(general), causal & (key_times[None] > times[:, None] - window))
                np.testing.assert_array_equal(general.view(np.uint8), mask.view(np.uint8))



def test_pinned_results_keep_their_dtype(monkeypatch):
    """``host.empty`` hands out arrays of the asked dtype, bfloat16 included (an array interface's typestr
    alone reads as raw two-byte items), backed by the leased block and returned to the pool when dropped."""
    import ctypes
    import gc

    from chroma_amd._src import host, native
    from chroma_amd._src.dtypes import BFLOAT16

    blocks = []

    class Library:
        def chroma_hip_host_alloc(self, size, handle, error, error_size):
            blocks.append(ctypes.create_string_buffer(size))
            ctypes.cast(handle, ctypes.POINTER(ctypes.c_void_p))[0] = ctypes.addressof(blocks[-1])
            return native.OK

    monkeypatch.setattr(native, "library", lambda: Library())
    monkeypatch.setattr(host, "_free", {})
    monkeypatch.setattr(host, "_held", 0)
    for dtype in (np.float32, BFLOAT16, np.int64):
        array = host.empty((3, 5), dtype)
        assert array.dtype == np.dtype(dtype) and array.shape == (3, 5) and array.flags.c_contiguous
        assert array.ctypes.data == ctypes.addressof(blocks[-1])
        array[...] = 1
        assert float(array.astype(np.float32).sum()) == 15.0
        del array
        gc.collect()
    assert host._free == {host.PAGE: [ctypes.addressof(blocks[0])]}  # one block, reused each time
    assert len(blocks) == 1
