"""The ``hip`` backend: a codegen plugin that emits gfx950 kernels and a launch plan.

It implements the plugin protocol the front end drives (the reference's ``Codegen`` surface,
chroma/_src/codegen/base.py:39-113 and gpu.py:63-435) and replaces the CUDA generator and its cuBLAS
calls (chroma/_src/codegen/cuda/codegen.py:44-168):

* A non-stored value is a closure ``(kernel, coordinates) -> node`` over the kernel compiler in
  ``kernel.py``; a consumer kernel inlines it. Materialisation happens when the front end asks for it,
  when an expression is 24 levels deep, or when it reads 24 buffers.
* Every launch is a deduplicated ``extern "C"`` kernel whose parameters are buffer base pointers; the
  plan binds each parameter to a region of the program's single device allocation (weights | workspace |
  error word | inputs | outputs), so the twelve identical layers of a model share their kernels.
* Whole-tensor operations (softmax, RMSNorm, reductions, top-k, linear, contractions) are generated
  around templates in ``csrc/include/chroma_hip`` and keep the reference CPU backend's numerics:
  float accumulation, division-based normalisation, RNE bfloat16 at every bfloat16 result, lowest-index
  tie-breaking in top-k with NaN ranked highest.
"""

from __future__ import annotations

import hashlib
import math
from dataclasses import dataclass, field
from typing import Callable, Dict, Iterator, List, Optional, Sequence, Set, Tuple, Union

import torch

from chroma_amd._src.codegen.base import Codegen, GeneratedCode
from chroma_amd._src.graph import fuse_attention
from chroma_amd._src.codegen.kernel import ZERO, Aff, Atom, Kernel, choose_lanes, ctype_of, float_literal, is_int
from chroma_amd._src.spec import Stats, TensorSpec, nbytes
from chroma_amd._src.value import ITEMSIZE, Value, View, contiguous_strides, contraction, matrix_axes

Closure = Callable[[Kernel, List[Aff]], tuple]

ALIGN = 256
MAX_DEPTH = 24
MAX_SOURCES = 24
MAP_THREADS = 256
MAX_GRID = 16384
# Elementwise (map and concatenation) kernels launch one thread per vector up to this many workgroups,
# so no thread walks a grid-stride loop and every load of the launch can be in flight at once.
MAP_GRID = 1 << 20
# Elementwise results of at most this many vectors with an outermost extent up to this many launch one
# workgroup row per outermost index.
SPLIT_MAP_VECTORS = 4096
SPLIT_MAP_ROWS = 1024
# Row kernels: threads per row for rows of at least 2048 elements (smaller rows use one wave), the most
# elements a thread keeps in registers for a single-pass row, and whether results that nothing in the
# same kernel reads again are written with non-temporal (streaming) stores.
ROW_THREADS = 256
ROW_RESIDENT = 32
ROW_UNROLL = 4  # vector loads per thread in flight in the one-pass row statistics
# a row softmax whose row splits evenly into at least two vector steps of this many threads takes them: fewer
# values per thread leave more waves resident (C2's [16384, 8192] fp32 rows: 2-3% faster than 256 threads,
# measured in one process)
WIDE_ROW_THREADS = 1024
SPLIT_ROW_LIMIT = 256  # rows of a reduction below this count are split over workgroups when wide
SPLIT_ROW_BLOCKS = 1024  # workgroups a split row reduction aims for
COOP_THREADS = 1024  # threads of a cooperative row kernel's workgroup (one workgroup per compute unit)
COOP_GROUPS = 64  # rows in flight at most (chroma::kCoopGroups counter words)
STREAMING_STORES = True
STREAMING_BYTES = 64 << 20  # smaller operands and results may stay in L2 / the last-level cache
FUSED_CONCAT_ELEMENTS = 1 << 16  # smaller concatenations are fused into their consumers
DEFERRED_ELEMENTS = 1 << 16  # smaller expressions the front end asks to store stay fused instead...
DEFERRED_SOURCES = 4  # ...when they read at most this many buffers (a residual stream is stored every few adds)
CHEAP_EXPRESSION_COST = 8  # larger expressions stay fused too when one element costs at most this much
WIDE_TOPK_LANE_VALUES = 32  # rows needing more values per lane take the two-stage top-k
TRANSCENDENTAL_OPS = frozenset({"sin", "cos", "exp", "tanh", "sigmoid", "silu", "pow", "log"})
STORED_TABLE_ELEMENTS = 4096  # multi-consumer expressions with such ops and at least this many elements are stored
MFMA_CUS = 256  # compute units of the target (MI355X), for the tile-round choice of the matrix-core products
DIRECT_GEMM_THREADS = 512  # chroma::kDirectThreads: the direct-to-LDS matrix-core body's 8 waves
# minimum resident workgroups per compute unit it is compiled for (__launch_bounds__'s second argument):
# two 64 KiB-LDS workgroups of 8 waves, i.e. 4 waves per SIMD and up to 128 VGPRs each
DIRECT_GEMM_BLOCKS = 2
WIDE_GEMM_THREADS = 256  # chroma::kWideThreads: the wide matrix-core body's 4 waves, one 140 KiB-LDS workgroup per CU
WIDE_GEMM_TILE = (256, 192)  # chroma::kWideM, kWideN
# the wide body takes dense products with at least this many of its tiles: below that its larger tiles
# leave too much of the chip idle and the 128 x 128 body is faster
WIDE_GEMM_MIN_TILES = 200
# below that, products with at least this many 128 x 192 tiles take the mid ring body (chroma::kMidThreads
# 4 waves, one 100 KiB-LDS workgroup per CU); smaller ones the 128 x 128 direct body
MID_GEMM_TILE = (128, 192)  # chroma::kMidM, kMidN
MID_GEMM_THREADS = 256
MID_GEMM_MIN_TILES = 160
MID_GEMMS = True
# A matrix-core linear (other than the wide body) whose weights (a constant) take this many bytes or more, up
# to a quarter of the 256 MB memory-side cache, is preceded by a launch that reads them (chroma::prefetch_bytes):
# its copy ring then finds them in that cache instead of waiting an HBM round trip per stage
PREFETCH_WEIGHT_BYTES = (4 << 20, 64 << 20)
PREFETCH_BLOCKS = 2048
WEIGHT_PREFETCH = True
# bfloat16 expert products whose channel count is a multiple of a tile width here (the first that fits)
# take the ring body (chroma::grouped_expert_linear PATH 3) on 128-slot x width tiles with that many waves
# side by side (each wave all slots of a width / waves strip), and an expert's last tile holds up to the
# third figure's slots: at 160 a remainder of up to 32 slots past a full tile joins it instead of costing
# a whole tile of its own (chroma::kTallLastTile). Measured on the GPT-OSS-20B shapes (2048 tokens x top-4
# of 32): with balanced routing (~256 slots per expert, half the experts with a third tile of a few slots)
# the 5760-channel up product on 384 x 8 waves takes 466 us with 128-slot last tiles and 409 us with 160;
# the 2880-channel down product on 320 x 4 waves 240 us and 250 us (its 585 workgroups still take three
# rounds of the chip's 256, now with longer tiles among them), on 192 x 4 waves with 160 236 us, but 276 us
# against 241 us on the skewed routing the seeded C5 model produces (expert counts 0-1842 at layer 19).
RING_EXPERT_TILES = ((384, 8, 160), (320, 4, 128))
# A gated activation between two expert products is computed in the first product's epilogue (no map
# launch; the first product is not stored when nothing else reads it). False keeps the separate launch.
ACTIVATION_EPILOGUES = True
# An elementwise expression of a row-per-workgroup RMSNorm's output (the workloads' cast to bfloat16) is
# written by the norm kernel itself. False keeps the separate map launch.
NORM_EPILOGUES = True
# A stored map reading only weights and graph inputs is launched once per distinct kernel and bindings
# (``_constant_map``). False launches every one.
CONSTANT_MAPS = True
# A concatenation of equal parts along the innermost dimension writes every part's element at one position from
# one thread (``_concat_kernel``). False keeps one part per thread.
PAIRED_CONCAT = True
REUSED_EVALUATIONS = 1 << 18  # a contraction operand is stored when (elements x reuse) reaches this
SMALL_REDUCTION = 8  # contractions summing at most this many products are fused expressions...
SMALL_OPERAND_COST = 8  # ...over operands that cost at most this much per element (others are stored)
MATRIX_MIN_WORK = 1 << 18  # smaller batched products stay on the generic contraction kernel
GROUPED_SLOTS = 64  # from this many (token, expert) slots on, expert products are grouped by expert
FUSED_ROUTER_BYTES = 32 << 10  # a router with gate weights up to this size is recomputed inside its first expert product
EARLY_FETCH_BYTES = 1 << 20  # weight streams up to this size are requested before their staging prologue
ROUTER_TICKETS = 48  # rows a split router can serve (chroma::kRouterTickets words of the error region)
ERROR_REGION = 1024  # bytes of the error region: error word, router tickets, decode-attention tickets
ATTENTION_TICKETS = 64  # (query row, head) rows a split-key decode attention can serve (chroma::kAttentionTickets)
NARROW_COLUMNS = 64  # linears of at most this many columns over many rows take one workgroup per 16 rows
SMALL_INPUT_BYTES = 64 << 10  # inputs up to this size are staged ahead of the larger ones
MATRIX_ATTENTION_TOKENS = 64  # bfloat16 attention over at least this many queries runs on the matrix cores
# query heads per wave of the grouped prefill attention (attention_heads): two share each K and V^T fragment
# read from LDS, whose bandwidth bounds the one-head form; compiled for 3 resident workgroups per compute unit
# (164 registers: unbounded it takes 204 and 2 fit, at 4 it spills). C5 full layer 132 -> 125 us standalone,
# a 4-layer prefill slice 5.945 -> 5.890 ms, bit-identical
ATTENTION_HEADS_PER_WAVE = 2
# the live-tile table of a mask whose rows are whole 16-byte chunks is built by one wave per tile
# (chroma::attention_live_tiles_wave) instead of a 256-thread workgroup
WAVE_LIVE_TILES = True
ATTENTION_HEADS_MIN_BLOCKS = 3
SPLIT_KEYS = 256  # keys per workgroup when an attention row's keys are split over workgroups
DECODE_SPLIT_KEYS = 128  # the same for stored key/value rows read with 16-byte loads (decode steps)
WAVE_ATTENTION_KEYS = 1024  # up to this many keys, attention runs one wave per query head
STREAM_BLOCKS = 2048  # workgroups of a weight-streaming product (4-8 per compute unit keep HBM busy)
SPREAD_BYTES = 8 << 20  # weight-streaming products up to this size take one row step per wave
STAGED_FLOATS = 8192  # X rows up to this many floats are widened into LDS once per workgroup
# ...and up to this many for a weight-streaming linear (128 KiB of LDS, one workgroup per compute unit):
# C1's 8 x 4096 down product streams its weights there with X (and its fused SiLU x up) read from LDS,
# 46.6 -> 36.2 us for the block, where the register-blocked skinny product spilled
LINEAR_STAGED_FLOATS = 32768
STAGED_ROWS = 4096  # new key/value rows of an attention up to this many floats are evaluated into LDS once
FOLDED_NORM_ROWS = 16  # RMSNorms over at most this many rows are folded into the kernels that stage them
LDS_STAGED_FLOATS = 12288  # floats a staging prologue may keep in LDS (X rows and evaluated operands)
SPLIT_STAGING_TRIPS = 8  # staging loops of at least this many trips request every trip's loads first...
STAGED_LOAD_REGISTERS = 128  # ...when those loads fit this many registers
FOLDED_STAGING_BLOCKS = 1024  # staging kernels with more workgroups read a stored copy of an expression operand

UNARY_OPS = {
    "reciprocal": "reciprocal",
    "rsqrt": "rsqrt",
    "sigmoid": "sigmoid",
    "sin": "sin",
    "cos": "cos",
    "exp": "exp",
    "neg": "neg",
    "abs": "abs",
    "square": "square",
    "tanh": "tanh",
    "silu": "silu",
    "log": "log",
}


@dataclass(frozen=True)
class Binding:
    kind: str  # "weight" | "arena" | "input" | "output" | "error"
    index: Union[int, str] = 0  # input/output position, or arena allocation name
    offset: int = 0  # byte offset (weights: inside the blob)


@dataclass
class Launch:
    kernel: str
    grid: Tuple[int, int, int]
    block: int
    bindings: List[Binding]
    shared: int = 0
    buffers: List[str] = field(default_factory=list)  # the buffers behind ``bindings``


def _align(value: int) -> int:
    return -(-value // ALIGN) * ALIGN


def _shape(value_shape: Sequence[int]) -> Tuple[int, ...]:
    return tuple(value_shape) if value_shape else (1,)


class _NotFusible(Exception):
    """An epilogue fusion does not apply to this expression (the plain launches are kept)."""


class HIPCodegen(Codegen):
    backend = "hip"
    graph_passes = (fuse_attention,)

    def __init__(self, *, blas: bool = True) -> None:
        super().__init__()
        self.blas = blas
        self.closures: Dict[str, Closure] = {}
        self.costs: Dict[str, int] = {}
        self.transcendental: Set[str] = set()  # expressions containing a libm call
        self.sources: Dict[str, frozenset] = {}
        self.bindings: Dict[str, Binding] = {}
        self.dtypes: Dict[str, torch.dtype] = {}
        self.kernel_names: Dict[str, str] = {}
        self.kernel_sources: List[str] = []
        self.launches: List[Launch] = []
        self.gathers: Dict[str, Tuple[Value, Value]] = {}
        self.routes: Dict[Tuple[str, int], Value] = {}
        self.extents: Dict[str, int] = {}
        self.parallel_reductions = 0
        self.expert_contractions = 0
        self.tiled_matmuls = 0
        self.skinny_matmuls = 0
        self.mfma_matmuls = 0
        self.fused_attentions = 0
        self.attention_epilogues = 0
        self.retractable_attention: Dict[str, tuple] = {}  # wave attention output -> (launch index, operands, inputs)
        self.small_contractions = 0
        self.live_block_tables: Dict[tuple, Value] = {}
        self.pending_norms: Dict[str, tuple] = {}  # deferred RMSNorm value -> (meta, x, weight, epsilon)
        self.pending_of: Dict[str, frozenset] = {}  # value -> deferred norms its expression reads
        self.retractable: Dict[str, tuple] = {}  # small linear output -> (launch index, x, weight, bias)
        self.router_weights: Dict[str, Value] = {}  # top-k values -> their softmax, written by the router
        self.router_launches: Dict[str, dict] = {}  # router indices -> the router launch (for fusion into its expert product)
        self.routed_experts = 0  # routers fused into their first expert product
        # Write-through stores: a small expression the front end asks to store gets its arena buffer at
        # once, but the buffer is written by the first kernel that reads it. A staging kernel computes the
        # expression itself and also stores it; any other reader has a copy kernel launched before it.
        self.store_expressions: Dict[str, Value] = {}  # arena buffer -> the expression it holds
        self.pending_stores: Set[str] = set()  # buffers not written yet
        self.resolved_by_launch: Dict[int, List[str]] = {}  # launch index -> buffers that launch writes
        self.write_through_stores: Set[str] = set()  # buffers written by the first kernel that stages them
        self.folded_norms = 0
        self.fused_routers = 0
        # Gated activations computed in the epilogue of the expert product they read: the last grouped ring
        # launch (to re-emit with an epilogue), the activations' stored copies (expression -> buffer), and
        # per fused launch (launch index, product buffer, the variant that does not store the product),
        # swapped in at the end when nothing else reads the product.
        self.last_grouped: Optional[dict] = None
        self.epilogue_values: Dict[str, Value] = {}
        self.product_stores: List[Tuple[int, str, Kernel, Tuple[int, int, int], int, Sequence[str], str]] = []
        self.expert_epilogues = 0
        self.unstored_products = 0
        self.constant_maps: Dict[tuple, Value] = {}  # (kernel, read bindings, grid) -> buffer it wrote
        self.reused_maps = 0
        self.last_norm: Optional[dict] = None  # the last one-workgroup-per-row RMSNorm launch
        self.norm_epilogues = 0
        self.weight_prefetches = 0

    # ===================================================================================== storage
    def extern(self, tensor: torch.Tensor, kind: str, offset: int) -> Value:
        name = f"v{next(self.counter)}"
        shape = tuple(tensor.shape)
        self.bindings[name] = Binding("input", offset) if kind == "input" else Binding("weight", 0, offset)
        self.dtypes[name] = tensor.dtype
        self.sources[name] = frozenset({name})
        self.extents[name] = math.prod(shape)
        return Value(name, shape, tensor.dtype, stored=True, view=View(None, contiguous_strides(shape)))

    def allocate(self, shape, dtype) -> Value:
        value = super().allocate(shape, dtype)
        self.bindings[value.name] = Binding("arena", value.name)
        self.dtypes[value.name] = dtype
        self.sources[value.name] = frozenset({value.name})
        self.extents[value.name] = math.prod(value.shape)
        return value

    def alias(self, meta: torch.Tensor, root: Value, offset: int) -> Value:
        shape = tuple(meta.shape)
        name = f"v{next(self.counter)}"
        self.sources[name] = self.sources[root.name]
        return Value(name, shape, meta.dtype, root.deps, stored=True, view=View(root, contiguous_strides(shape), offset))

    # ================================================================================= expressions
    def expr(self, meta: torch.Tensor, closure: Closure, inputs: Sequence[Value], cost: Optional[int] = None,
             transcendental: bool = False) -> Value:
        name = f"e{next(self.counter)}"
        self.closures[name] = closure
        # rough count of the loads and operations one element costs (stored inputs count one load)
        self.costs[name] = cost if cost is not None else 1 + sum(self.cost(v) for v in inputs)
        if transcendental or any(v.name in self.transcendental for v in inputs if not v.stored):
            self.transcendental.add(name)
        self.sources[name] = frozenset().union(*(self.sources[v.name] for v in inputs)) if inputs else frozenset()
        pending = frozenset().union(*(self.pending_of.get(v.name, frozenset()) for v in inputs)) if inputs else frozenset()
        if pending:
            self.pending_of[name] = pending
        value = self.expression_value(name, meta, inputs)
        if value.depth >= MAX_DEPTH or len(self.sources[name]) >= MAX_SOURCES:
            return self.store(value)
        return value

    def cost(self, value: Value) -> int:
        return 1 if value.stored else self.costs.get(value.name, 1)

    def read(self, k: Kernel, value: Value, coords: Sequence[Aff]) -> tuple:
        """The node for ``value`` at ``coords`` (one affine coordinate per dimension)."""
        staged = k.staged_values.get(value.name)
        if staged is not None:
            return ("lds", staged, Kernel.flatten(coords, _shape(value.shape)) if value.shape else ZERO)
        stored_copy = self.epilogue_values.get(value.name)
        if stored_copy is not None:
            return self.read(k, stored_copy, coords)
        if value.stored:
            root, view = value.root, value.view
            address = Aff((), view.offset)
            for coord, stride, size in zip(coords, view.strides, value.shape):
                if size != 1 and stride:
                    address = address + coord.scale(stride)
            hook = k.register_reads.get(root.name)
            if hook is not None:
                return hook(address)
            if root.name in k.staged_values:
                return ("lds", k.staged_values[root.name], address)
            expression = k.unstored.get(root.name)
            if expression is not None:
                if value.name == root.name:
                    return self.read(k, expression, coords)
                return self.read(k, expression, k.unflatten(address, expression.shape))
            return ("ld", k.slot(root.name, root.dtype, extent=self.extents[root.name]), value.dtype, address)
        key = (value.name, tuple(coords))
        node = k.values.get(key)
        if node is None:
            node = self.closures[value.name](k, list(coords))
            k.values[key] = node
        return node

    def read_flat(self, k: Kernel, value: Value, flat: Aff) -> tuple:
        if (value.stored and value.view.base is None and value.name not in k.unstored and value.name not in k.staged_values
                and value.name not in k.register_reads):
            return ("ld", k.slot(value.name, value.dtype, extent=self.extents[value.name]), value.dtype, flat)
        return self.read(k, value, k.unflatten(flat, value.shape))

    def broadcast_read(self, k: Kernel, value: Value, coords: Sequence[Aff], shape: Sequence[int]) -> tuple:
        pad = len(shape) - len(value.shape)
        mine = [ZERO if size == 1 else coords[d + pad] for d, size in enumerate(value.shape)]
        return self.read(k, value, mine)

    def materialize(self, value: Value) -> Value:
        """The front end's request to store ``value`` (``clone``/``contiguous``, or an elementwise result
        with several consumers). Values are immutable, so storage is a performance decision here:

        * a strided view of a stored buffer already has storage and is returned as one (consumers read it
          through its strides; matrix kernels ask for ``contiguous`` instead);
        * an expression of at most ``DEFERRED_ELEMENTS`` elements reading at most ``DEFERRED_SOURCES``
          buffers stays fused into each consumer, where it costs a few instructions instead of a launch
          (consumers evaluate shared subexpressions once); longer chains, such as a residual stream over
          many layers, are stored so that no consumer re-evaluates the whole chain;
        * anything larger is written to the arena once.
        """
        if value.stored:
            return value
        if value.view is not None and value.view.base is not None:
            return Value(value.name, value.shape, value.dtype, value.deps, stored=True, view=value.view)
        if value.name in self.pending_norms:
            return value  # consumers that stage their rows fold it; any other reader stores it
        if value.name in self.transcendental and STORED_TABLE_ELEMENTS <= math.prod(value.shape) <= DEFERRED_ELEMENTS:
            # a table of libm calls (the rotary cos/sin at a long prefill) that several consumers read,
            # typically broadcast over heads: computed once instead of once per consumer element
            return self.store(value)
        if math.prod(value.shape) <= DEFERRED_ELEMENTS and len(self.sources[value.name]) <= DEFERRED_SOURCES:
            return value
        if math.prod(value.shape) > DEFERRED_ELEMENTS and value.name in self.closures and self.cost(value) <= CHEAP_EXPRESSION_COST:
            # a large elementwise result that costs a few loads per element: each consumer re-reading its
            # sources moves fewer bytes than writing it and reading it back
            return value
        if self.blas and value.name in self.closures and value.name not in self.materialized and math.prod(value.shape) <= STAGED_FLOATS:
            out = self.allocate(value.shape, value.dtype)
            self.materialized[value.name] = out
            self.store_expressions[out.name] = value
            self.pending_stores.add(out.name)
            return out
        return self.store(value)

    def _flush_store(self, buffer: str) -> None:
        """Write a pending write-through buffer with a copy kernel (launched before its reader)."""
        self.pending_stores.discard(buffer)
        value = self.store_expressions[buffer]
        self.map_kernel(self.materialized[value.name], value)

    def store(self, value: Value) -> Value:
        """Write ``value`` to a fresh arena allocation (once; later requests reuse it)."""
        if value.stored:
            return value
        if value.name in self.pending_norms:
            return self._force_norm(value.name)
        if value.name not in self.materialized:
            fused = self._norm_epilogue(value)
            self.materialized[value.name] = fused if fused is not None else self._constant_map(self.allocate(value.shape, value.dtype), value)
        return self.materialized[value.name]

    def _norm_epilogue(self, value: Value) -> Optional[Value]:
        """Store ``value`` from the RMSNorm kernel that is the last launch when ``value`` is an elementwise
        expression of that norm's output (same shape; any other buffer it reads is a weight or graph
        input): the norm launch is re-emitted writing ``value`` too, and, unless some later launch reads
        the norm itself, finally without the norm's store. The workloads' norms end with a cast to
        bfloat16, which then costs no map launch and no float round trip."""
        last = self.last_norm
        if not NORM_EPILOGUES or last is None or last["index"] != len(self.launches) - 1 or value.stored or value.name not in self.closures:
            return None
        out, x, weight, epsilon = last["args"]
        sources = self.sources.get(value.name, frozenset())
        if (out.name not in sources or tuple(value.shape) != tuple(out.shape)
                or any(self.binding_of(b).kind not in ("weight", "input") for b in sources if b != out.name)):
            return None
        buffer = self.allocate(tuple(value.shape), value.dtype)
        try:
            k, prologue = self._rmsnorm_rows(out, x, weight, epsilon, epilogue=(value, buffer))
            lean, _ = self._rmsnorm_rows(out, x, weight, epsilon, epilogue=(value, buffer), store_norm=False)
        except _NotFusible:
            return None
        self._retract_last_launch()
        self.launch(k, last["rows"], last["threads"], [x, weight, value], kind="rmsnorm", prologue=prologue)
        self.product_stores.append((len(self.launches) - 1, out.root.name, lean, self.launches[-1].grid, last["threads"], prologue, "rmsnorm"))
        self.epilogue_values[value.name] = buffer
        self.last_norm = None
        self.norm_epilogues += 1
        return buffer

    def _constant_map(self, out: Value, value: Value) -> Value:
        """``map_kernel(out, value)``, except that a map reading only weights and graph inputs (which no
        launch writes) whose kernel and bindings equal an earlier one's is not launched again: the earlier
        buffer already holds the same values and is returned instead (the per-layer rotary cos/sin
        tables of a prefill are computed once)."""
        shape = _shape(value.shape)
        lanes = choose_lanes(shape[-1], value.dtype, 8 if value.dtype == torch.bfloat16 else 4)
        k, grid = self._map_kernel(out, value, None, lanes)
        if lanes == 8 and k.scalar_lane_loads:
            k, grid = self._map_kernel(out, value, None, 4)
        reads = [buffer for buffer in k.slots if buffer != out.name]
        key = None
        if CONSTANT_MAPS and all(self.binding_of(buffer).kind in ("weight", "input") for buffer in reads):
            key = (k.render("KERNEL_NAME", MAP_THREADS), tuple(self.binding_of(buffer) for buffer in reads), grid)
            earlier = self.constant_maps.get(key)
            if earlier is not None:
                self.reused_maps += 1
                return earlier
        self.launch(k, grid, MAP_THREADS, [value], kind="map")
        if key is not None:
            self.constant_maps[key] = out
        return out

    @staticmethod
    def is_contiguous(value: Value) -> bool:
        if not value.stored:
            return False
        natural = contiguous_strides(value.shape)
        return all(size == 1 or a == b for size, a, b in zip(value.shape, value.view.strides, natural))

    def contiguous(self, value: Value) -> Value:
        """A stored, row-major copy of ``value`` (the value itself when it already is one)."""
        if self.is_contiguous(value):
            return value
        key = value.name + "#contiguous"
        if key not in self.materialized:
            out = self._norm_epilogue(value)
            if out is None:
                out = self.allocate(value.shape, value.dtype)
                self.map_kernel(out, value)
            self.materialized[key] = out
        return self.materialized[key]

    def reshape(self, meta: torch.Tensor, x: Value) -> Value:
        if self.is_contiguous(x):
            return self.alias(meta, x.root, x.view.offset)
        shape = tuple(meta.shape)

        def closure(k: Kernel, coords: List[Aff]) -> tuple:
            return self.read_flat(k, x, Kernel.flatten(coords, shape))

        return self.expr(meta, closure, [x])

    def reindex(self, meta: torch.Tensor, x: Value, mapping: Sequence[int], offset: int) -> Value:
        shape = tuple(meta.shape)

        def closure(k: Kernel, coords: List[Aff]) -> tuple:
            flat = Aff((), offset)
            for coord, stride, size in zip(coords, mapping, shape):
                if size != 1 and stride:
                    flat = flat + coord.scale(stride)
            return self.read_flat(k, x, flat)

        return self.expr(meta, closure, [x])

    def cast(self, meta: torch.Tensor, x: Value) -> Value:
        to_bf16 = meta.dtype == torch.bfloat16 and x.dtype != torch.bfloat16

        def closure(k: Kernel, coords: List[Aff]) -> tuple:
            node = self.read(k, x, coords)
            return ("rnd", node) if to_bf16 else node

        return self.expr(meta, closure, [x])

    def elementwise(self, meta, target: str, args, *, alpha: float = 1, low: Optional[float] = None, high: Optional[float] = None) -> Value:
        shape = tuple(meta.shape)
        op = target.split(".")[1]
        bf16 = meta.dtype == torch.bfloat16

        def rounded(node: tuple) -> tuple:
            return ("rnd", node) if bf16 else node

        def closure(k: Kernel, coords: List[Aff]) -> tuple:
            def operand(a) -> tuple:
                return self.broadcast_read(k, a, coords, shape) if isinstance(a, Value) else ("f", float(a))

            a = operand(args[0])
            if op in ("add", "sub"):
                b = operand(args[1])
                if alpha != 1:
                    b = rounded(("bin", "mul", b, ("f", float(alpha))))
                node = ("bin", op, a, b)
            elif op == "rsub":
                node = ("bin", "sub", operand(args[1]), rounded(("bin", "mul", a, ("f", float(alpha)))))
            elif op in ("mul", "div"):
                node = ("bin", op, a, operand(args[1]))
            elif op == "pow":
                b = operand(args[1])
                node = ("un", "square", a) if b == ("f", 2.0) else ("bin", "pow", a, b)
            elif op == "clamp":
                node = a
                if low is not None:
                    node = ("bin", "lowclamp", node, ("f", float(low)))
                if high is not None:
                    node = ("bin", "highclamp", node, ("f", float(high)))
            else:
                node = ("un", UNARY_OPS[op], a)
            return rounded(node)

        return self.expr(meta, closure, [v for v in args if isinstance(v, Value)], transcendental=op in TRANSCENDENTAL_OPS)

    def gather(self, meta, x: Value, indices: Value, negative: bool) -> Value:
        index_rank = len(indices.shape)
        rows = x.shape[0]

        def closure(k: Kernel, coords: List[Aff]) -> tuple:
            selected = self.read(k, indices, coords[:index_rank])
            row = k.index_atom(selected, rows, negative)
            return self.read(k, x, [row, *coords[index_rank:]])

        value = self.expr(meta, closure, [x, indices])
        if negative and not value.stored:
            self.gathers[value.name] = (x, indices)
        return value

    def triangular(self, meta, x: Value, diagonal: int, upper: bool) -> Value:
        zero = ("i", 0) if is_int(meta.dtype) else ("f", 0.0)

        def closure(k: Kernel, coords: List[Aff]) -> tuple:
            keep = ("cmp", ">=" if upper else "<=", coords[-1], coords[-2], int(diagonal))
            return ("sel", keep, self.read(k, x, coords), zero)

        return self.expr(meta, closure, [x])

    # ================================================================================= launching
    def binding_of(self, buffer: str) -> Binding:
        return self.bindings[buffer]

    def launch(
        self,
        k: Kernel,
        grid: Union[int, Tuple[int, int, int]],
        block: int,
        inputs: Sequence[Value],
        *,
        kind: str,
        prologue: Sequence[str] = (),
        shared: int = 0,
    ) -> None:
        """Record one launch of ``k``; identical kernels (same code, same parameter types) are emitted once.

        Kernels are named ``chroma_<kind>_<hash of their source>`` so profiles stay readable and
        stable across programs."""
        for buffer in list(k.slots):
            if buffer in self.pending_stores and buffer not in k.unstored:
                self._flush_store(buffer)
        for buffer, (_, _, writable) in k.slots.items():
            # weights and graph inputs are never written by a launch (``_constant_map`` relies on it)
            if writable and self.binding_of(buffer).kind in ("weight", "input"):
                raise AssertionError(f"a launch writes {buffer}, a weight or graph input")
        source = k.render("KERNEL_NAME", block, prologue)
        name = self.kernel_names.get(source)
        if name is None:
            name = f"chroma_{kind}_{hashlib.sha256(source.encode()).hexdigest()[:8]}"
            self.kernel_names[source] = name
            self.kernel_sources.append(source.replace("KERNEL_NAME", name, 1))
        grid3 = (grid, 1, 1) if isinstance(grid, int) else grid
        if any(g > 2**31 - 1 for g in grid3):
            raise ValueError("HIP dispatch exceeds the grid limit")
        bindings = [self.binding_of(buffer) for buffer in k.slots]
        for buffer in k.slots:
            allocation = self.allocations.get(buffer)
            if allocation is not None:
                # live at every launch that touches it (a fused launch may take the index of an earlier one)
                allocation.start = min(allocation.start, self.kernels)
                allocation.end = max(allocation.end, self.kernels)
        self.record_usage(inputs)
        self.launches.append(Launch(name, grid3, block, bindings, shared, list(k.slots)))
        if k.resolved_stores:
            self.resolved_by_launch[len(self.launches) - 1] = list(k.resolved_stores)
        self.kernels += 1

    def map_kernel(self, out: Value, value: Value, target: Optional[str] = None) -> None:
        """out[i] = value[i] over a contiguous destination (an allocation or an output region). bfloat16
        results take 8 lanes per thread (16-byte accesses) unless some operand could not be read that
        wide; then 4."""
        shape = _shape(value.shape)
        lanes = choose_lanes(shape[-1], value.dtype, 8 if value.dtype == torch.bfloat16 else 4)
        k, grid = self._map_kernel(out, value, target, lanes)
        if lanes == 8 and k.scalar_lane_loads:
            k, grid = self._map_kernel(out, value, target, 4)
        self.launch(k, grid, MAP_THREADS, [value], kind="map")

    def _map_kernel(self, out: Value, value: Value, target: Optional[str], lanes: int) -> Tuple[Kernel, Union[int, Tuple[int, int, int]]]:
        shape = _shape(value.shape)
        count = math.prod(shape)
        k = Kernel(lanes)
        k.streaming = STREAMING_STORES and count * ITEMSIZE[value.dtype] >= STREAMING_BYTES
        k.streaming_loads = STREAMING_BYTES if k.streaming else 0
        slot = k.slot(target or out.name, value.dtype, writable=True, extent=self.extents[target or out.name])
        vectors = count // lanes
        vshape = shape[:-1] + (shape[-1] // lanes,)
        # A small result gets one workgroup per outermost index: that index is then uniform, so a
        # concatenation along it (stacked per-layer results) evaluates one part per workgroup instead of
        # every part in one wave.
        split = len(shape) > 1 and 1 < shape[0] <= SPLIT_MAP_ROWS and vectors <= SPLIT_MAP_VECTORS
        if split:
            outer = Aff.of(k.atom("blockIdx.y", shape[0] - 1))
            vshape = vshape[1:]
            vectors //= shape[0]
        wide = vectors > 2**31 - 1
        itype = "uint64_t" if wide else "uint32_t"
        loop = f"for ({itype} v = {itype}(blockIdx.x) * {MAP_THREADS}u + threadIdx.x; v < {vectors}u; v += {itype}(gridDim.x) * {MAP_THREADS}u) {{"
        with k.block(loop):
            v = Atom("v", vectors - 1)
            coords = ([outer] if split else []) + k.unflatten(Aff.of(v), vshape)
            if lanes > 1:
                coords[-1] = Aff.of(k.vector_atom(f"({coords[-1].code()}) * {lanes}u", shape[-1] - 1))
            node = self.read(k, value, coords if value.shape else coords[:0])
            k.store(slot, value.dtype, Kernel.flatten(coords, shape), node)
        grid = max(1, min(-(-vectors // MAP_THREADS), MAP_GRID))
        return k, ((grid, shape[0], 1) if split else grid)

    # ==================================================================================== outputs
    def output(self, index: int, value: Value) -> None:
        if value.stored and value.root.name in self.pending_stores:
            self._flush_store(value.root.name)
        if self.promote_output(index, value):
            return
        name = f"output{index}"
        self.bindings[name] = Binding("output", index)
        self.dtypes[name] = value.dtype
        self.extents[name] = math.prod(value.shape)
        out = Value(name, value.shape, value.dtype, stored=True, view=View(None, contiguous_strides(value.shape)))
        self.map_kernel(out, value, target=name)

    # =================================================================================== concat
    def concatenate(self, meta, values: Sequence[Value], dim: int) -> Value:
        if math.prod(meta.shape) <= FUSED_CONCAT_ELEMENTS:
            return self._concat_expression(meta, values, dim)
        out = self.allocate(tuple(meta.shape), meta.dtype)
        shape = _shape(out.shape)
        innermost = dim == len(shape) - 1
        # bfloat16 parts take 8 lanes (16-byte accesses) like the map kernels, unless some operand could not
        # be read that wide; then 4
        lanes = choose_lanes(shape[-1], meta.dtype, 8 if meta.dtype == torch.bfloat16 else 4)
        if innermost:
            while lanes > 1 and any(v.shape[dim] % lanes for v in values):
                lanes //= 2
        k, grid = self._concat_kernel(out, values, dim, lanes)
        if lanes == 8 and k.scalar_lane_loads:
            k, grid = self._concat_kernel(out, values, dim, 4)
        self.launch(k, grid, MAP_THREADS, values, kind="concat")
        return out

    def _concat_kernel(self, out: Value, values: Sequence[Value], dim: int, lanes: int) -> Tuple[Kernel, int]:
        shape = _shape(out.shape)
        innermost = dim == len(shape) - 1
        count = math.prod(shape)
        k = Kernel(lanes)
        slot = k.slot(out.name, out.dtype, writable=True, extent=self.extents[out.name])
        size = values[0].shape[dim]
        if (PAIRED_CONCAT and innermost and lanes > 1 and len(values) > 1 and size % lanes == 0
                and all(value.shape[dim] == size for value in values)):
            # Equal parts along the innermost dimension (the two halves of a rotary embedding): a thread
            # writes the same position of every part, so what the parts read in common (x1, x2, cos, sin)
            # is loaded once.
            vectors = count // lanes // len(values)
            with k.block(f"for (uint32_t v = blockIdx.x * {MAP_THREADS}u + threadIdx.x; v < {vectors}u; v += gridDim.x * {MAP_THREADS}u) {{"):
                v = Atom("v", vectors - 1)
                coords = k.unflatten(Aff.of(v), shape[:-1] + (size // lanes,))
                coords[-1] = Aff.of(k.vector_atom(f"({coords[-1].code()}) * {lanes}u", size - 1))
                for i, value in enumerate(values):
                    node = self.read(k, value, coords)
                    k.store(slot, out.dtype, Kernel.flatten(coords[:-1] + [coords[-1] + i * size], shape), node)
            return k, max(1, min(-(-vectors // MAP_THREADS), MAP_GRID))
        vectors = count // lanes
        with k.block(f"for (uint32_t v = blockIdx.x * {MAP_THREADS}u + threadIdx.x; v < {vectors}u; v += gridDim.x * {MAP_THREADS}u) {{"):
            v = Atom("v", vectors - 1)
            vshape = shape[:-1] + (shape[-1] // lanes,)
            coords = k.unflatten(Aff.of(v), vshape)
            if lanes > 1:
                coords[-1] = Aff.of(k.vector_atom(f"({coords[-1].code()}) * {lanes}u", shape[-1] - 1))
            along = coords[dim]
            along_code = k.atom(along.code(), shape[dim] - 1, prefix="c") if not innermost or lanes == 1 else None
            start = 0
            for i, value in enumerate(values):
                end = start + value.shape[dim]
                if innermost and lanes > 1:
                    test = f"{coords[-1].code()} < {end}u"
                else:
                    test = f"{along_code.name} < {end}u"
                opener = ("if (" if i == 0 else "} else if (") + test + ") {" if i < len(values) - 1 else ("} else {" if i else "{")
                k.line(opener)
                k.indent += 1
                saved = (dict(k.atoms), dict(k.nodes), dict(k.values))
                local = list(coords)
                if innermost and lanes > 1:
                    local[dim] = Aff.of(k.vector_atom(f"{coords[dim].code()} - {start}u", value.shape[dim] - 1))
                else:
                    local[dim] = Aff.of(k.atom(f"{along_code.name} - {start}u", value.shape[dim] - 1, prefix="c"))
                node = self.read(k, value, local)
                k.store(slot, out.dtype, Kernel.flatten(coords, shape), node)
                k.atoms, k.nodes, k.values = saved
                k.indent -= 1
                start = end
            k.line("}")
        return k, max(1, min(-(-vectors // MAP_THREADS), MAP_GRID))

    def _concat_expression(self, meta, values: Sequence[Value], dim: int) -> Value:
        """Concatenation folded into its consumer: a case split over the parts along ``dim`` (only the
        selected part is evaluated when the position along ``dim`` is the same for every lane of a thread;
        otherwise every part is evaluated and selected). Coordinates are clamped into each part's range,
        so no read leaves its buffer either way."""
        starts = [0]
        for value in values:
            starts.append(starts[-1] + value.shape[dim])

        def closure(k: Kernel, coords: List[Aff]) -> tuple:
            along = coords[dim]
            parts, tests = [], []
            for i in range(len(values)):
                start, size = starts[i], values[i].shape[dim]
                local = list(coords)
                local[dim] = k.derived(along, f"({{0}}) < {start}u ? 0u : (({{0}}) - {start}u < {size}u ? ({{0}}) - {start}u : {size - 1}u)", size - 1)
                parts.append(self.read(k, values[i], local))
                if i < len(values) - 1:
                    tests.append(("cmp", "<", along, ZERO, starts[i + 1]))
            return ("cases", tuple(tests), tuple(parts))

        return self.expr(meta, closure, list(values))

    # ================================================================================ row kernels
    def _row_layout(self, shape: Sequence[int], dim: int) -> Tuple[int, int, int]:
        width = shape[dim]
        inner = math.prod(shape[dim + 1 :])
        outer = math.prod(shape[:dim])
        return width, inner, outer

    def _row_coords(self, k: Kernel, row: Aff, shape: Sequence[int], dim: int, along: Aff) -> List[Aff]:
        """Coordinates of element ``along`` of row ``row`` (rows enumerate outer x inner positions)."""
        inner_shape = tuple(shape[dim + 1 :])
        inner = math.prod(inner_shape)
        outer_coords = k.unflatten(k.div(row, inner), tuple(shape[:dim])) if dim else []
        inner_coords = k.unflatten(k.mod(row, inner), inner_shape) if inner_shape else []
        return [*outer_coords, along, *inner_coords]

    topk_width_limit = 64 * 64 * 64  # rows up to this wide: the two-stage selection below

    def _wide_topk(self, meta, x: Value, dim: int, largest: bool, values: Value, indices: Value) -> None:
        """Top-k of rows too wide to hold in one wave's registers (a vocabulary row of logits). Stage 1: one
        wave per chunk of 64 x P elements (at most 64 chunks per row) selects its chunk's k largest keys
        in order into a scratch list. Stage 2: one wave per row, lane c holding the head of chunk c's list,
        takes the wave-wide largest head k times. Keys order by value, then by lower index first
        (``topk_key``), and are unique, so the result is the single-pass selection's bit for bit."""
        shape = tuple(x.shape)
        width, inner, outer = self._row_layout(shape, dim)
        count = meta[0].shape[dim]
        rows = outer * inner
        per_lane = -(-width // (64 * 64))
        if per_lane > 64:
            raise NotImplementedError(f"topk over rows of {width} elements (at most {64 * 64 * 64})")
        chunk = 64 * per_lane
        chunks = -(-width // chunk)
        keys = self.allocate((rows * chunks * count,), torch.int64)
        vals = self.allocate((rows * chunks * count,), torch.float32)
        groups = 4
        k = Kernel(1)
        key_slot = k.slot(keys.name, torch.int64, writable=True, extent=self.extents[keys.name])
        val_slot = k.slot(vals.name, torch.float32, writable=True, extent=self.extents[vals.name])
        k.line(f"const uint32_t w = blockIdx.x * {groups}u + threadIdx.x / 64u;")
        k.line(f"if (w >= {rows * chunks}u) return;")
        k.line(f"const uint32_t r = w / {chunks}u, c = w % {chunks}u;")
        k.line("const uint32_t lane = threadIdx.x % 64u;")
        k.line(f"uint64_t keys[{per_lane}];")
        k.line(f"float vals[{per_lane}];")
        row = Aff.of(Atom("r", rows - 1))
        k.line("#pragma unroll")
        with k.block(f"for (uint32_t p = 0; p < {per_lane}u; ++p) {{"):
            k.line(f"const uint32_t j = c * {chunk}u + p * 64u + lane;")
            k.line(f"if (j < {width}u) {{")
            k.indent += 1
            j = Aff.of(Atom("j", width - 1))
            name = k.emit(self.read(k, x, self._row_coords(k, row, shape, dim, j)))
            k.line(f"vals[p] = {name}; keys[p] = chroma::topk_key({name}, j, {str(bool(largest)).lower()});")
            k.indent -= 1
            k.line("} else { vals[p] = 0.0f; keys[p] = 0; }")
        with k.block(f"for (uint32_t s = 0; s < {count}u; ++s) {{"):
            k.line("uint64_t best = 0;")
            k.line("#pragma unroll")
            k.line(f"for (uint32_t p = 0; p < {per_lane}u; ++p) best = keys[p] > best ? keys[p] : best;")
            k.line("const uint64_t top = chroma::wave_max_u64(best);")
            k.line(f"const size_t at = (size_t(r) * {chunks}u + c) * {count}u + s;")
            k.line("if (top == 0) { if (lane == 0) { " + key_slot + "[at] = 0; " + val_slot + "[at] = 0.0f; } continue; }")
            k.line("const uint32_t winner = 0xffffffffu - uint32_t(top);")
            k.line(f"if ((winner - c * {chunk}u) % 64u == lane) {{")
            k.indent += 1
            k.line("float chosen = 0.0f;")
            k.line("#pragma unroll")
            k.line(f"for (uint32_t p = 0; p < {per_lane}u; ++p) if (p == (winner - c * {chunk}u) / 64u) {{ chosen = vals[p]; keys[p] = 0; }}")
            k.line(f"{key_slot}[at] = int64_t(top); {val_slot}[at] = chosen;")
            k.indent -= 1
            k.line("}")
        self.launch(k, -(-(rows * chunks) // groups), 64 * groups, [x], kind="topk_chunks")

        k = Kernel(1)
        key_slot = k.slot(keys.name, torch.int64, extent=self.extents[keys.name])
        val_slot = k.slot(vals.name, torch.float32, extent=self.extents[vals.name])
        value_slot = k.slot(values.name, values.dtype, writable=True, extent=self.extents[values.name])
        index_slot = k.slot(indices.name, indices.dtype, writable=True, extent=self.extents[indices.name])
        k.line(f"const uint32_t r = blockIdx.x * {groups}u + threadIdx.x / 64u;")
        k.line(f"if (r >= {rows}u) return;")
        k.line("const uint32_t lane = threadIdx.x % 64u;")
        k.line(f"const size_t base = (size_t(r) * {chunks}u + lane) * {count}u;")
        k.line("uint32_t head = 0;")
        k.line(f"uint64_t key = lane < {chunks}u ? uint64_t({key_slot}[base]) : 0;")
        with k.block(f"for (uint32_t s = 0; s < {count}u; ++s) {{"):
            k.line("const uint64_t top = chroma::wave_max_u64(key);")
            k.line("if (top != 0 && key == top) {")
            k.indent += 1
            k.line(f"const float chosen = {val_slot}[base + head];")
            s_atom = Aff.of(Atom("s", count - 1))
            out_coords = self._row_coords(k, Aff.of(Atom("r", rows - 1)), tuple(meta[0].shape), dim, s_atom)
            address = Kernel.flatten(out_coords, tuple(meta[0].shape))
            k.store(value_slot, values.dtype, address, self._lane_values(k, ["chosen"]))
            k.line(f"{index_slot}[{address.code()}] = int64_t(0xffffffffu - uint32_t(top));")
            k.line("++head;")
            k.line(f"key = head < {count}u ? uint64_t({key_slot}[base + head]) : 0;")
            k.indent -= 1
            k.line("}")
        self.launch(k, -(-rows // groups), 64 * groups, [keys, vals], kind="topk_merge")

    def softmax(self, meta, x: Value, dim: int) -> Value:
        """Row softmax (gpu.py:275-298). The statistics are float, as in the reference; the quotient is
        exp(x - max) times the float reciprocal of the row's sum, one multiply per element instead of a
        division (a correctly rounded division costs about ten VALU operations, which would make the C2
        chain compute-bound), which keeps every result within one ulp of the correctly rounded quotient."""
        routed = self.router_weights.get(x.name)
        if routed is not None and dim == len(x.shape) - 1 and routed.dtype == meta.dtype:
            return routed
        out = self.allocate(tuple(meta.shape), meta.dtype)
        shape = tuple(x.shape)
        width, inner, outer = self._row_layout(shape, dim)
        rows = outer * inner
        if inner == 1 and width >= 64:
            splits, chunk, lanes = self._row_splits(rows, width, x.dtype)
            coop = self._coop_plan(rows, width, x.dtype, "softmax")
            if coop is not None and not self._row_plan(width, x.dtype, softmax=True)[3]:
                self._coop_rows("softmax", out, x, shape, dim, width, rows, coop)
            elif splits > 1 and not self._row_plan(width, x.dtype, softmax=True)[3]:
                self._split_softmax(out, x, shape, dim, width, rows, splits, chunk, lanes)
            else:
                self._row_softmax(out, x, shape, dim, width, rows)
            self.parallel_reductions += 1
        else:
            self._thread_softmax(out, x, shape, dim, width, rows)
        return out

    def _row_plan(self, width: int, dtype: torch.dtype, softmax: bool = False) -> Tuple[int, int, int, bool]:
        threads = ROW_THREADS if width >= 2048 else 64
        lanes = choose_lanes(width, dtype)
        if softmax and width % (WIDE_ROW_THREADS * lanes) == 0 and width >= 2 * WIDE_ROW_THREADS * lanes:
            threads = WIDE_ROW_THREADS
        chunks = -(-width // (threads * lanes))
        resident = chunks * lanes <= ROW_RESIDENT
        return threads, lanes, chunks, resident

    def _row_softmax(self, out: Value, x: Value, shape, dim: int, width: int, rows: int) -> None:
        threads, lanes, chunks, resident = self._row_plan(width, x.dtype, softmax=True)
        waves = threads // 64
        k = Kernel(lanes)
        k.streaming = STREAMING_STORES and math.prod(shape) * ITEMSIZE[out.dtype] >= STREAMING_BYTES
        k.streaming_loads = STREAMING_BYTES if k.streaming else 0
        slot = k.slot(out.name, out.dtype, writable=True, extent=self.extents[out.name])
        row_atom = k.atom("blockIdx.x", rows - 1, prefix="r")
        row = Aff.of(row_atom)
        step = threads * lanes
        ragged = width % step != 0
        neg_inf = float_literal(-math.inf)

        def element(j: Aff) -> tuple:
            return self.read(k, x, self._row_coords(k, row, shape, dim, j))

        def out_address(j: Aff) -> Aff:
            return Kernel.flatten(self._row_coords(k, row, shape, dim, j), shape)

        def lane_names(node) -> List[str]:
            names = k.emit(node)
            return names if isinstance(names, list) else [names] * lanes

        if resident:
            k.line(f"float vals[{chunks}][{lanes}];")
            k.line(f"float peak = {neg_inf};")
            if not ragged:
                k.load_replay = self._hoist_loads(k, chunks, lambda: lane_names(element(Aff.of(k.vector_atom(f"c * {step}u + threadIdx.x * {lanes}u", width - 1)))))
            k.line("#pragma unroll")
            with k.block(f"for (uint32_t c = 0; c < {chunks}u; ++c) {{"):
                j = Aff.of(k.vector_atom(f"c * {step}u + threadIdx.x * {lanes}u", width - 1))
                guard = ragged
                if guard:
                    k.line(f"if ({j.code()} < {width}u) {{")
                    k.indent += 1
                names = lane_names(element(j))
                for lane, name in enumerate(names):
                    k.line(f"vals[c][{lane}] = {name}; peak = __builtin_fmaxf(peak, {name});")
                if guard:
                    k.indent -= 1
                    k.line("} else {")
                    k.line("    " + " ".join(f"vals[c][{lane}] = {neg_inf};" for lane in range(lanes)))
                    k.line("}")
            k.load_replay = None
            k.line(f"peak = chroma::block_max<{waves}>(peak, scratch);")
            k.line("float total = 0.0f;")
            k.line("#pragma unroll")
            k.line(f"for (uint32_t c = 0; c < {chunks}u; ++c) {{")
            k.line(f"    #pragma unroll")
            k.line(f"    for (uint32_t l = 0; l < {lanes}u; ++l) {{ vals[c][l] = chroma::fast_exp(vals[c][l] - peak); total += vals[c][l]; }}")
            k.line("}")
            k.line(f"total = chroma::block_sum<{waves}>(total, scratch);")
            k.line("const float inverse = 1.0f / total;")
            k.line("#pragma unroll")
            with k.block(f"for (uint32_t c = 0; c < {chunks}u; ++c) {{"):
                j = Aff.of(k.vector_atom(f"c * {step}u + threadIdx.x * {lanes}u", width - 1))
                if ragged:
                    k.line(f"if ({j.code()} < {width}u) {{")
                    k.indent += 1
                result = self._lane_values(k, [f"vals[c][{lane}] * inverse" for lane in range(lanes)])
                k.store(slot, out.dtype, out_address(j), result)
                if ragged:
                    k.indent -= 1
                    k.line("}")
        else:
            k.line(f"float peak = {neg_inf}, total = 0.0f;")
            with k.block(f"for (uint32_t base = threadIdx.x * {lanes}u; base < {width}u; base += {step}u) {{"):
                j = Aff.of(k.vector_atom("base", width - 1))
                for name in lane_names(element(j)):
                    k.line(f"{{ const float top = __builtin_fmaxf(peak, {name});")
                    k.line(f"  total = top == {neg_inf} ? 0.0f : total * chroma::fast_exp(peak - top) + chroma::fast_exp({name} - top);")
                    k.line("  peak = top; }")
            k.line(f"const float row_peak = chroma::block_max<{waves}>(peak, scratch);")
            k.line(f"total = chroma::block_sum<{waves}>(peak == {neg_inf} ? 0.0f : total * chroma::fast_exp(peak - row_peak), scratch);")
            k.line("const float inverse = 1.0f / total;")
            with k.block(f"for (uint32_t base = threadIdx.x * {lanes}u; base < {width}u; base += {step}u) {{"):
                j = Aff.of(k.vector_atom("base", width - 1))
                names = lane_names(element(j))
                result = self._lane_values(k, [f"chroma::fast_exp({name} - row_peak) * inverse" for name in names])
                k.store(slot, out.dtype, out_address(j), result)
        self.launch(k, rows, threads, [x], kind="softmax_rows", prologue=[f"__shared__ float scratch[{max(waves, 1)}];"])

    @staticmethod
    def _hoist_loads(k: Kernel, chunks: int, body: Callable[[], object]) -> Optional[Iterator[str]]:
        """Issue every chunk's vector loads before any arithmetic: ``body`` (one chunk of a row, indexed by
        ``c``) is emitted once in a loop that keeps its vector loads in per-chunk register arrays (the
        arithmetic it also emits has no use and is dropped by the compiler). Returns the replay that makes
        the real pass read those arrays, or None (nothing emitted) when the body has side effects or
        no vector loads."""
        mark, uses_error = len(k.lines), k.uses_error
        k.load_log = []
        k.line("#pragma unroll")
        with k.block(f"for (uint32_t {k.load_index} = 0; {k.load_index} < {chunks}u; ++{k.load_index}) {{"):
            body()
        log, k.load_log = k.load_log, None
        if not log or k.uses_error != uses_error:
            del k.lines[mark:]
            k.uses_error = uses_error
            return None
        k.lines[mark:mark] = ["    " * k.indent + f"{vtype} {array}[{chunks}];" for array, vtype in log]
        # Keep the instruction scheduler from sinking the loads back to their uses.
        k.line("__builtin_amdgcn_sched_barrier(0);")
        return iter([array for array, _ in log])

    def _lane_values(self, k: Kernel, codes: Sequence[str]) -> tuple:
        """A varying node whose lane l is the C expression ``codes[l]`` (declared now)."""
        names = [k.fresh("q") for _ in codes]
        for name, code in zip(names, codes):
            k.line(f"const float {name} = {code};")
        node = ("raw", tuple(names))
        k.nodes[node] = names if k.lanes > 1 else names[0]
        return node

    def _thread_softmax(self, out: Value, x: Value, shape, dim: int, width: int, rows: int) -> None:
        k = Kernel(1)
        slot = k.slot(out.name, out.dtype, writable=True, extent=self.extents[out.name])
        neg_inf = float_literal(-math.inf)
        with k.block(f"for (uint32_t r = blockIdx.x * 256u + threadIdx.x; r < {rows}u; r += gridDim.x * 256u) {{"):
            row = Aff.of(Atom("r", rows - 1))
            j_atom = Atom("j", width - 1)

            def element() -> tuple:
                return self.read(k, x, self._row_coords(k, row, shape, dim, Aff.of(j_atom)))

            k.line(f"float peak = {neg_inf};")
            with k.block(f"for (uint32_t j = 0; j < {width}u; ++j) {{"):
                k.line(f"peak = __builtin_fmaxf(peak, {k.emit(element())});")
            k.line("float total = 0.0f;")
            with k.block(f"for (uint32_t j = 0; j < {width}u; ++j) {{"):
                k.line(f"total += chroma::fast_exp({k.emit(element())} - peak);")
            k.line("const float inverse = 1.0f / total;")
            with k.block(f"for (uint32_t j = 0; j < {width}u; ++j) {{"):
                value = self._lane_values(k, [f"chroma::fast_exp({k.emit(element())} - peak) * inverse"])
                k.store(slot, out.dtype, Kernel.flatten(self._row_coords(k, row, shape, dim, Aff.of(j_atom)), shape), value)
        self.launch(k, max(1, min(-(-rows // 256), MAX_GRID)), 256, [x], kind="softmax_lines")

    # -------------------------------------------------------------------------------- row statistics
    # A row's softmax statistics in one HBM pass: each thread keeps an online maximum ``peak``, the sum
    # ``total`` of exp(x - peak) over the elements it read (rescaled when the maximum grows) and a NaN
    # flag; the workgroup then combines its threads'. Rows too few to fill the chip are split over
    # workgroups (``_row_partials``), whose (peak, total) pairs a later launch combines in the same way.

    @staticmethod
    def _coop_plan(rows: int, width: int, dtype: torch.dtype, kind: str) -> Optional[Tuple[int, int, int]]:
        """(parts per row, vectors per thread, lanes) of a cooperative row kernel, or None: rows too wide for
        one workgroup's registers and many enough to fill the chip (``SPLIT_ROW_LIMIT``); each of ``parts``
        workgroups of ``COOP_THREADS`` holds ``vectors`` vectors of ``lanes`` per thread (at most 6: three
        rows in registers at once, and for an RMSNorm its slice of the weight), the parts covering the row
        with at most 1/16 of it as padding."""
        if dtype not in (torch.float32, torch.bfloat16) or rows < SPLIT_ROW_LIMIT:
            return None
        lanes = choose_lanes(width, dtype)
        if width % lanes:
            return None
        step = COOP_THREADS * lanes
        most = 6
        best = None
        for parts in range(2, 17):
            vectors = -(-width // (parts * step))
            if vectors > most or (parts - 1) * vectors * step >= width:
                continue
            waste = parts * vectors * step - width
            if waste * 16 <= width and (best is None or waste < best[0]):
                best = (waste, parts, vectors)
        return None if best is None else (best[1], best[2], lanes)

    def _coop_rows(self, kind: str, out: Value, x: Value, shape, dim: int, width: int, rows: int, plan: Tuple[int, int, int],
                   weight: Optional[Value] = None, epsilon: float = 0.0) -> None:
        """One HBM pass of a wide row softmax (gpu.py:275-298) or RMSNorm (gpu.py:339-358) over many rows: a
        persistent grid of ``parts`` x groups co-resident workgroups (one per compute unit), group g taking
        rows g, g + groups, ...; each part keeps its slice of a row in registers and publishes its partial
        statistics (softmax: the slice's maximum, NaN if it holds a NaN, and sum of exp(x - max); RMSNorm:
        its sum of squares) with ``chroma::coop_publish``; one row later (so the exchange overlaps a row of
        work) it collects the other parts' statistics of that row (``coop_peek``, ``coop_wait``), requests
        its slice of the row after next, combines the statistics in part order and writes its slice: exp(x - max)
        times the reciprocal of the sum (NaN for a row holding a NaN, a +inf or only -inf, as in
        ``_split_softmax``), or x * (1 / sqrt(sum / D + eps)) * w."""
        parts, vectors, lanes = plan
        threads = COOP_THREADS
        step = threads * lanes
        span = vectors * step
        groups = max(1, min(MFMA_CUS // parts, rows, COOP_GROUPS))
        floats = 2 if kind == "softmax" else 1
        words = 4 * parts * floats  # 64-bit words per group: four slot sets of each part's floats
        slots = self.allocate((groups * words * 2,), torch.float32)
        neg_inf = float_literal(-math.inf)
        k = Kernel(lanes)
        k.streaming = STREAMING_STORES and math.prod(shape) * ITEMSIZE[out.dtype] >= STREAMING_BYTES
        k.uses_error = True
        k.min_waves = 1
        slot = k.slot(out.name, out.dtype, writable=True, extent=self.extents[out.name])
        slot_buffer = k.slot(slots.name, torch.float32, writable=True, extent=self.extents[slots.name])
        waves = threads // 64
        k.line(f"const uint32_t group = blockIdx.x / {parts}u, part = blockIdx.x % {parts}u;")
        k.line(f"const uint32_t begin = part * {span}u + threadIdx.x * {lanes}u;")
        k.line(f"unsigned long long* const slots = reinterpret_cast<unsigned long long*>({slot_buffer}) + group * {words}u;")
        k.line(f"float cur[{vectors}][{lanes}], nxt[{vectors}][{lanes}], ahead[{vectors}][{lanes}];")

        def element_index(v: str) -> str:
            return f"begin + {v} * {step}u"

        def load(row_code: str, array: str) -> None:
            """``array`` <- the part's slice of row ``row_code`` (padding past the row's end)."""
            with k.block("{"):
                row = Aff.of(k.atom(row_code, rows - 1, prefix="r"))
                k.line("#pragma unroll")
                with k.block(f"for (uint32_t v = 0; v < {vectors}u; ++v) {{"):
                    k.line(f"const uint32_t at = {element_index('v')};")
                    j = Aff.of(k.vector_atom(f"at < {width}u ? at : {width - lanes}u", width - 1))
                    names = k.emit(self.read(k, x, self._row_coords(k, row, shape, dim, j)))
                    names = names if isinstance(names, list) else [names] * lanes
                    for lane, name in enumerate(names):
                        k.line(f"{array}[v][{lane}] = {name};")  # past the row's end: a copy of its last vector

        def over_slice(statement: str) -> None:
            """``statement`` for every element of the slice; ``live`` says whether it lies inside the row
            (the loads are unconditional, so the padding is applied where the values are used)."""
            k.line("#pragma unroll")
            k.line(f"for (uint32_t v = 0; v < {vectors}u; ++v) {{")
            k.line(f"    const bool live = {element_index('v')} < {width}u;")
            k.line("    #pragma unroll")
            k.line(f"    for (uint32_t l = 0; l < {lanes}u; ++l) {{ {statement} }}")
            k.line("}")

        if kind == "rmsnorm":
            k.line(f"float wv[{vectors}][{lanes}];")
            k.line("#pragma unroll")
            with k.block(f"for (uint32_t v = 0; v < {vectors}u; ++v) {{"):
                k.line(f"const uint32_t at = {element_index('v')};")
                j = Aff.of(k.vector_atom(f"at < {width}u ? at : {width - lanes}u", width - 1))
                names = k.emit(self.read(k, weight, [j]))
                names = names if isinstance(names, list) else [names] * lanes
                for lane, name in enumerate(names):
                    k.line(f"wv[v][{lane}] = {name};")
        # rows of this group: group, group + groups, ...; round r publishes row r's statistics (``nxt``),
        # collects round r - 1's, requests row r + 1 (``ahead``) and writes row r - 1 (``cur``): each
        # exchange overlaps a row of work, and the next row's loads overlap the writing
        k.line(f"const uint32_t count = ({rows}u - group + {groups - 1}u) / {groups}u;")
        load("group", "nxt")
        k.line("bool ok = true;")
        with k.block("for (uint32_t round = 0; round <= count && ok; ++round) {"):
            with k.block("if (round < count) {"):
                if kind == "softmax":
                    k.line(f"float peak = {neg_inf};")
                    k.line("bool bad = false;")
                    over_slice(f"peak = __builtin_fmaxf(peak, live ? nxt[v][l] : {neg_inf}); bad = bad | (live && __builtin_isnan(nxt[v][l]));")
                    k.line(f"peak = chroma::block_max<{waves}>(peak, scratch);")
                    k.line("float total = 0.0f;")
                    with k.block(f"if (peak != {neg_inf}) {{"):
                        over_slice("total += live ? chroma::fast_exp(nxt[v][l] - peak) : 0.0f;")
                    k.line(f"total = chroma::block_sum<{waves}>(total, scratch);")
                    k.line(f"const bool flagged = chroma::block_max<{waves}>(bad ? 1.0f : 0.0f, scratch) != 0.0f;")
                    k.line('const float mine[2] = {flagged ? __builtin_nanf("") : peak, total};')
                else:
                    k.line("float squares = 0.0f;")
                    over_slice("squares += live ? nxt[v][l] * nxt[v][l] : 0.0f;")
                    k.line(f"const float mine[1] = {{chroma::block_sum<{waves}>(squares, scratch)}};")
                k.line(f"chroma::coop_publish<{parts}, {floats}>(slots, part, round, mine);")
            # round r - 1 was published a row ago: its words are normally there at the first look, so only
            # the peek's round trip is exposed; the next row's loads are requested after the check (a check
            # after them would wait for them too) and overlap the writing of row r - 1
            k.line(f"float all[{parts}][{floats}];")
            with k.block("if (round > 0) {"):
                k.line(f"const unsigned long long word = chroma::coop_peek<{parts}, {floats}>(slots, round - 1u);")
                k.line(f"ok = chroma::coop_wait<{parts}, {floats}>(slots, round - 1u, word, all, error);")
            with k.block("if (round + 1u < count) {"):
                load(f"group + (round + 1u) * {groups}u", "ahead")
            with k.block("if (round > 0) {"):
                if kind == "softmax":
                    k.line(f"float row_peak = {neg_inf}, row_total = 0.0f;")
                    k.line("bool row_bad = false;")
                    k.line("#pragma unroll")
                    k.line(f"for (uint32_t q = 0; q < {parts}u; ++q) {{ row_peak = __builtin_fmaxf(row_peak, all[q][0]); row_bad = row_bad | __builtin_isnan(all[q][0]); }}")
                    k.line("#pragma unroll")
                    k.line(f"for (uint32_t q = 0; q < {parts}u; ++q) row_total += all[q][0] == {neg_inf} || __builtin_isnan(all[q][0]) ? 0.0f : "
                           "all[q][1] * chroma::fast_exp(all[q][0] - row_peak);")
                    k.line('const float inverse = row_bad || __builtin_isinf(row_peak) ? __builtin_nanf("") : 1.0f / row_total;')
                else:
                    k.line("float row_squares = 0.0f;")
                    k.line("#pragma unroll")
                    k.line(f"for (uint32_t q = 0; q < {parts}u; ++q) row_squares += all[q][0];")
                    k.line(f"const float scale = 1.0f / sqrtf(row_squares / {float_literal(width)} + {float_literal(epsilon)});")
                row = Aff.of(k.atom(f"group + (round - 1u) * {groups}u", rows - 1, prefix="r"))
                k.line("#pragma unroll")
                with k.block(f"for (uint32_t v = 0; v < {vectors}u; ++v) {{"):
                    k.line(f"const uint32_t at = {element_index('v')};")
                    with k.block(f"if (at < {width}u) {{"):
                        j = Aff.of(k.vector_atom("at", width - 1))
                        if kind == "softmax":
                            codes = [f"chroma::fast_exp(cur[v][{lane}] - row_peak) * inverse" for lane in range(lanes)]
                        else:
                            codes = [f"cur[v][{lane}] * scale * wv[v][{lane}]" for lane in range(lanes)]
                        k.store(slot, out.dtype, Kernel.flatten(self._row_coords(k, row, shape, dim, j), shape), self._lane_values(k, codes))
            over_slice("cur[v][l] = nxt[v][l]; nxt[v][l] = ahead[v][l];")
        k.line(f"chroma::coop_depart<{parts}, {floats}>(slots, error + chroma::kCoopDepartWord + group);")
        inputs = [x] + ([weight] if weight is not None else [])
        self.launch(k, parts * groups, threads, inputs, kind=f"coop_{kind}", prologue=[f"__shared__ float scratch[{waves}];"])

    @staticmethod
    def _row_splits(rows: int, width: int, dtype: torch.dtype) -> Tuple[int, int, int]:
        """(splits per row, elements per split, lanes): one workgroup per row when there are at least
        ``SPLIT_ROW_LIMIT`` rows or a row is narrow; otherwise enough splits for about ``SPLIT_ROW_BLOCKS``
        workgroups, each at least ``ROW_UNROLL`` vectors per thread (one round of loads in flight)."""
        lanes = choose_lanes(width, dtype, 8 if dtype == torch.bfloat16 else 4)
        step = ROW_THREADS * lanes
        if rows >= SPLIT_ROW_LIMIT or width < 2 * ROW_UNROLL * step:
            return 1, width, lanes
        wanted = -(-SPLIT_ROW_BLOCKS // rows)
        chunk = -(-(-(-width // wanted)) // step) * step
        chunk = max(chunk, ROW_UNROLL * step)
        return -(-width // chunk), chunk, lanes

    def _row_stats(self, k: Kernel, x: Value, shape, dim: int, row: Aff, width: int, begin: str, end: str) -> None:
        """Declare ``row_peak``, ``row_total`` and ``row_bad`` (1 when a NaN was read) for elements [begin,
        end) of row ``row`` (``begin`` a multiple of the workgroup's step; ``end`` a multiple of the lanes).
        ``ROW_UNROLL`` vector loads per thread are requested before their arithmetic."""
        lanes, threads = k.lanes, ROW_THREADS
        step = threads * lanes
        neg_inf = float_literal(-math.inf)

        def names_of(j: Aff) -> List[str]:
            names = k.emit(self.read(k, x, self._row_coords(k, row, shape, dim, j)))
            return names if isinstance(names, list) else [names] * lanes

        def accumulate(names: List[str]) -> None:
            level = list(names)
            while len(level) > 1:
                level = [f"__builtin_fmaxf({a}, {b})" for a, b in zip(level[::2], level[1::2])] + level[len(level) // 2 * 2 :]
            terms = " + ".join(f"chroma::fast_exp({name} - top)" for name in names)
            k.line(f"{{ const float top = __builtin_fmaxf(peak, {level[0]});")
            k.line("  bad = bad | " + " | ".join(f"__builtin_isnan({name})" for name in names) + ";")
            k.line(f"  if (top != {neg_inf}) total = total * chroma::fast_exp(peak - top) + ({terms});")
            k.line("  peak = top; }")

        k.line(f"float peak = {neg_inf}, total = 0.0f;")
        k.line("bool bad = false;")
        k.line(f"uint32_t base = {begin} + threadIdx.x * {lanes}u;")
        with k.block(f"for (; base + {(ROW_UNROLL - 1) * step}u < {end}; base += {ROW_UNROLL * step}u) {{"):
            groups = [names_of(Aff.of(k.vector_atom(f"base + {u * step}u", width - 1))) for u in range(ROW_UNROLL)]
            for names in groups:
                accumulate(names)
        with k.block(f"for (; base < {end}; base += {step}u) {{"):
            accumulate(names_of(Aff.of(k.vector_atom("base", width - 1))))
        waves = threads // 64
        k.line(f"const float row_peak = chroma::block_max<{waves}>(peak, scratch);")
        k.line(f"const float row_total = chroma::block_sum<{waves}>(peak == {neg_inf} ? 0.0f : total * chroma::fast_exp(peak - row_peak), scratch);")
        k.line(f"const bool row_bad = chroma::block_max<{waves}>(bad ? 1.0f : 0.0f, scratch) != 0.0f;")

    def _row_partials(self, x: Value, shape, dim: int, width: int, rows: int, splits: int, chunk: int, lanes: int) -> Value:
        """One workgroup per (row, split): the split's (peak, total) into a float pair of a scratch buffer;
        a split that read a NaN stores NaN as its peak."""
        partials = self.allocate((rows * splits * 2,), torch.float32)
        k = Kernel(lanes)
        slot = k.slot(partials.name, torch.float32, writable=True, extent=self.extents[partials.name])
        row = Aff.of(k.atom(f"blockIdx.x / {splits}u", rows - 1, prefix="r"))
        k.line(f"const uint32_t begin = blockIdx.x % {splits}u * {chunk}u;")
        k.line(f"const uint32_t end = begin + {chunk}u < {width}u ? begin + {chunk}u : {width}u;")
        self._row_stats(k, x, shape, dim, row, width, "begin", "end")
        k.line("if (threadIdx.x == 0) {")
        k.line(f"    {slot}[2u * blockIdx.x] = row_bad ? __builtin_nanf(\"\") : row_peak;")
        k.line(f"    {slot}[2u * blockIdx.x + 1u] = row_total;")
        k.line("}")
        self.launch(k, rows * splits, ROW_THREADS, [x], kind="row_partials", prologue=[f"__shared__ float scratch[{ROW_THREADS // 64}];"])
        return partials

    @staticmethod
    def _combine_partials(k: Kernel, slot: str, splits: int, first: str, stride: int, threads: int, reduce: str) -> None:
        """Declare ``row_peak``, ``row_total``, ``row_bad`` from the ``splits`` (peak, total) pairs at
        ``slot[2 * (first + s)]`` read by ``threads`` threads (``reduce``: "wave" or "block")."""
        neg_inf = float_literal(-math.inf)
        lane = "threadIdx.x % 64u" if reduce == "wave" else "threadIdx.x"
        k.line(f"float peak = {neg_inf}, total = 0.0f;")
        k.line("bool bad = false;")
        with k.block(f"for (uint32_t s = {lane}; s < {splits}u; s += {stride}u) {{"):
            k.line(f"const float p = {slot}[2u * ({first} + s)], t = {slot}[2u * ({first} + s) + 1u];")
            k.line("bad = bad | __builtin_isnan(p);")
            k.line("const float top = __builtin_fmaxf(peak, p);")
            k.line(f"if (top != {neg_inf}) total = total * chroma::fast_exp(peak - top) + (p == {neg_inf} || __builtin_isnan(p) ? 0.0f : t * chroma::fast_exp(p - top));")
            k.line("peak = top;")
        scaled = f"peak == {neg_inf} ? 0.0f : total * chroma::fast_exp(peak - row_peak)"
        if reduce == "wave":
            k.line("const float row_peak = chroma::wave_max(peak);")
            k.line(f"const float row_total = chroma::wave_sum({scaled});")
            k.line("const bool row_bad = chroma::wave_max(bad ? 1.0f : 0.0f) != 0.0f;")
        else:
            waves = threads // 64
            k.line(f"const float row_peak = chroma::block_max<{waves}>(peak, scratch);")
            k.line(f"const float row_total = chroma::block_sum<{waves}>({scaled}, scratch);")
            k.line(f"const bool row_bad = chroma::block_max<{waves}>(bad ? 1.0f : 0.0f, scratch) != 0.0f;")

    @staticmethod
    def _lse_of_stats() -> str:
        """C expression of torch's log-sum-exp from the row statistics: NaN if a NaN was read, +inf for a
        +inf maximum, -inf for an all -inf row, else log(total) + peak."""
        inf = float_literal(math.inf)
        return (f"row_bad ? __builtin_nanf(\"\") : (row_peak == {inf} ? {inf} : "
                f"(row_peak == -{inf} ? -{inf} : logf(row_total) + row_peak))")

    def _split_softmax(self, out: Value, x: Value, shape, dim: int, width: int, rows: int, splits: int, chunk: int, lanes: int) -> None:
        """Softmax of few wide rows (a vocabulary row of logits): ``_row_partials`` gives each split's
        statistics; then each (row, split) workgroup combines its row's pairs and writes its split of the
        row as exp(x - max) times the reciprocal of the sum (the second read of the split mostly hits the
        last-level cache). A row with a NaN, a +inf or only -inf gives NaN everywhere, as the reference's
        exp(x - max) / sum does."""
        partials = self._row_partials(x, shape, dim, width, rows, splits, chunk, lanes)
        k = Kernel(lanes)
        k.streaming = STREAMING_STORES and math.prod(shape) * ITEMSIZE[out.dtype] >= STREAMING_BYTES
        part_slot = k.slot(partials.name, torch.float32, extent=self.extents[partials.name])
        slot = k.slot(out.name, out.dtype, writable=True, extent=self.extents[out.name])
        row_atom = k.atom(f"blockIdx.x / {splits}u", rows - 1, prefix="r")
        row = Aff.of(row_atom)
        self._combine_partials(k, part_slot, splits, f"{row_atom.name} * {splits}u", ROW_THREADS, ROW_THREADS, "block")
        k.line('const float inverse = row_bad || __builtin_isinf(row_peak) ? __builtin_nanf("") : 1.0f / row_total;')
        k.line(f"const uint32_t begin = blockIdx.x % {splits}u * {chunk}u;")
        k.line(f"const uint32_t end = begin + {chunk}u < {width}u ? begin + {chunk}u : {width}u;")
        step = ROW_THREADS * lanes

        def write(j: Aff, names: List[str]) -> None:
            result = self._lane_values(k, [f"chroma::fast_exp({name} - row_peak) * inverse" for name in names])
            k.store(slot, out.dtype, Kernel.flatten(self._row_coords(k, row, shape, dim, j), shape), result)

        def names_of(j: Aff) -> List[str]:
            names = k.emit(self.read(k, x, self._row_coords(k, row, shape, dim, j)))
            return names if isinstance(names, list) else [names] * lanes

        k.line(f"uint32_t base = begin + threadIdx.x * {lanes}u;")
        with k.block(f"for (; base + {(ROW_UNROLL - 1) * step}u < end; base += {ROW_UNROLL * step}u) {{"):
            js = [Aff.of(k.vector_atom(f"base + {u * step}u", width - 1)) for u in range(ROW_UNROLL)]
            loaded = [names_of(j) for j in js]
            for j, names in zip(js, loaded):
                write(j, names)
        with k.block(f"for (; base < end; base += {step}u) {{"):
            j = Aff.of(k.vector_atom("base", width - 1))
            write(j, names_of(j))
        self.launch(k, rows * splits, ROW_THREADS, [x, partials], kind="softmax_split",
                    prologue=[f"__shared__ float scratch[{ROW_THREADS // 64}];"])

    # -------------------------------------------------------------------------------- log-sum-exp
    def logsumexp(self, meta, x: Value, dim: int) -> Value:
        """log(sum(exp(x))) along ``dim``: an extension (the reference's operator table has no
        ``aten.logsumexp``) with torch's definition: m = the maximum along the axis (0 when infinite),
        m + log(sum(exp(x - m))), float statistics, rounded once to the output type; a NaN element gives
        NaN and a +inf element (without NaN) +inf. Rows of 64 or more contiguous elements take one HBM pass
        (``_row_stats``): one workgroup per row, or, when there are fewer rows than fill the chip (a few
        vocabulary rows of logits), a split of each row over workgroups and a small combining launch."""
        out = self.allocate(tuple(meta.shape), meta.dtype)
        shape = tuple(x.shape)
        width, inner, outer = self._row_layout(shape, dim)
        rows = outer * inner
        if inner != 1 or width < 64:
            self._thread_lse(out, x, shape, dim, width, rows)
            return out
        splits, chunk, lanes = self._row_splits(rows, width, x.dtype)
        self.parallel_reductions += 1
        if splits == 1:
            k = Kernel(lanes)
            slot = k.slot(out.name, out.dtype, writable=True, extent=self.extents[out.name])
            row_atom = k.atom("blockIdx.x", rows - 1, prefix="r")
            self._row_stats(k, x, shape, dim, Aff.of(row_atom), width, "0u", f"{width}u")
            with k.block("if (threadIdx.x == 0) {"):
                k.store(slot, out.dtype, Aff.of(row_atom), self._lane_values(k, [self._lse_of_stats()]))
            self.launch(k, rows, ROW_THREADS, [x], kind="logsumexp_rows", prologue=[f"__shared__ float scratch[{ROW_THREADS // 64}];"])
            return out
        partials = self._row_partials(x, shape, dim, width, rows, splits, chunk, lanes)
        k = Kernel(1)
        part_slot = k.slot(partials.name, torch.float32, extent=self.extents[partials.name])
        slot = k.slot(out.name, out.dtype, writable=True, extent=self.extents[out.name])
        k.line("const uint32_t r = blockIdx.x * 4u + threadIdx.x / 64u;")
        k.line(f"if (r >= {rows}u) return;  // whole waves leave together")
        self._combine_partials(k, part_slot, splits, f"r * {splits}u", 64, 256, "wave")
        with k.block("if (threadIdx.x % 64u == 0) {"):
            k.store(slot, out.dtype, Aff.of(Atom("r", rows - 1)), self._lane_values(k, [self._lse_of_stats()]))
        self.launch(k, -(-rows // 4), 256, [partials], kind="logsumexp_combine")
        return out

    def _thread_lse(self, out: Value, x: Value, shape, dim: int, width: int, rows: int) -> None:
        """One thread per row (narrow or strided rows): the maximum, then the sum, then the result."""
        k = Kernel(1)
        slot = k.slot(out.name, out.dtype, writable=True, extent=self.extents[out.name])
        neg_inf = float_literal(-math.inf)
        with k.block(f"for (uint32_t r = blockIdx.x * 256u + threadIdx.x; r < {rows}u; r += gridDim.x * 256u) {{"):
            row = Aff.of(Atom("r", rows - 1))
            j_atom = Atom("j", width - 1)

            def element() -> tuple:
                return self.read(k, x, self._row_coords(k, row, shape, dim, Aff.of(j_atom)))

            k.line(f"float row_peak = {neg_inf};")
            k.line("bool row_bad = false;")
            with k.block(f"for (uint32_t j = 0; j < {width}u; ++j) {{"):
                name = k.emit(element())
                k.line(f"row_peak = __builtin_fmaxf(row_peak, {name}); row_bad = row_bad | __builtin_isnan({name});")
            k.line("const float shift = __builtin_isinf(row_peak) ? 0.0f : row_peak;")
            k.line("float row_total = 0.0f;")
            with k.block(f"for (uint32_t j = 0; j < {width}u; ++j) {{"):
                k.line(f"row_total += chroma::fast_exp({k.emit(element())} - shift);")
            k.store(slot, out.dtype, row, self._lane_values(k, [self._lse_of_stats()]))
        self.launch(k, max(1, min(-(-rows // 256), MAX_GRID)), 256, [x], kind="logsumexp_lines")

    # -------------------------------------------------------------------------------- RMSNorm
    def norm(self, meta, x: Value, weight: Value, epsilon: float) -> Value:
        """RMSNorm. A norm over at most ``FOLDED_NORM_ROWS`` rows is deferred: kernels that stage their
        operand rows in LDS (weight-streaming linears, selected experts, the router) compute the row
        scales in their prologue and apply ``x * scale * w`` while staging, so the normalised rows are
        never written; the first other reader stores it with the norm kernel below."""
        shape = _shape(x.shape)
        if math.prod(shape) // shape[-1] <= FOLDED_NORM_ROWS and self.blas:
            name = f"r{next(self.counter)}"
            value = Value(name, tuple(meta.shape), meta.dtype, x.deps | weight.deps, depth=1)
            self.pending_norms[name] = (meta, x, weight, epsilon)
            self.sources[name] = self.sources[x.name] | self.sources[weight.name]
            self.pending_of[name] = frozenset({name})
            self.closures[name] = lambda k, coords, name=name: self._norm_node(k, name, coords)
            return value
        return self._norm_kernel(meta, x, weight, epsilon)

    def _force_norm(self, name: str) -> Value:
        if name not in self.materialized:
            self.materialized[name] = self._norm_kernel(*self.pending_norms[name])
        return self.materialized[name]

    def _norm_node(self, k: Kernel, name: str, coords: Sequence[Aff]) -> tuple:
        """The deferred norm at ``coords``: from its stored copy if one exists, from the row scales a
        staging prologue declared in ``k``, or else by storing it now."""
        if name in self.materialized:
            return self.read(k, self.materialized[name], coords)
        scales = getattr(k, "norm_scales", {}).get(name)
        if scales is None:
            return self.read(k, self._force_norm(name), coords)
        meta, x, weight, _ = self.pending_norms[name]
        shape = _shape(x.shape)
        row = Kernel.flatten(list(coords[:-1]), shape[:-1]) if len(shape) > 1 else ZERO
        key = ("norm_scale", name, row)
        if key not in k.nodes:
            scale = k.fresh("s")
            k.line(f"const float {scale} = {scales}[{row.code()}];")
            k.nodes[key] = scale
        scale_node = ("raw", (k.nodes[key],))
        k.nodes[scale_node] = k.nodes[key]
        return ("bin", "mul", ("bin", "mul", self.read(k, x, coords), scale_node), self.read(k, weight, [coords[-1]]))

    def _stageable(self, x: Value, blocks: int) -> Value:
        """The operand a staging kernel of ``blocks`` workgroups should read: every workgroup evaluates
        the staged rows itself, so an expression (or a deferred norm) is stored once first when many
        workgroups would repeat it."""
        if blocks <= FOLDED_STAGING_BLOCKS or x.stored or (x.view is not None and x.view.base is not None):
            return x
        return self.store(x)

    def _stage(self, k: Kernel, x: Value, rows: int, inner: int, coords_of: Callable[[Aff], List[Aff]], threads: int, array: str = "xs") -> None:
        """Emit the prologue that fills ``__shared__ float array[rows * inner]`` with ``x`` row by row:
        element (r, c) is ``x`` at ``coords_of(r) + [c]``, evaluated through generated code (so views and
        fused expressions are read in place). Deferred norms that ``x`` depends on get their row scales
        computed first. Ends with a workgroup barrier. The prologue's threads exchange data through LDS only,
        so its barriers publish LDS alone and leave a weight stream requested before it in flight."""
        waves = threads // 64
        resolved = []
        for buffer in sorted((self.sources[x.name] & self.pending_stores) - set(k.slots)):
            # ``x`` reads a write-through buffer nothing has written yet: this kernel evaluates its
            # expression wherever it would load it, and the first workgroup also stores it. (A buffer
            # the kernel already reads through a pointer is left to the copy kernel instead.)
            k.unstored[buffer] = self.store_expressions[buffer]
            k.resolved_stores.append(buffer)
            self.pending_stores.discard(buffer)
            resolved.append(buffer)
            self.write_through_stores.add(buffer)  # (a retracted launch's buffers are resolved again by its replacement)
        budget = [LDS_STAGED_FLOATS - rows * inner]

        def staging_loop(count: int, element: Callable[[List[Aff]], object], shape: Sequence[int], target: str) -> None:
            """``target[i] = element(i)`` for the ``count`` staged elements. Element 0 is evaluated at the
            enclosing scope first, so row indices gathered through values that do not depend on the element
            (a token's id, the selected experts) are loaded and checked once instead of once per unrolled
            batch (the unused element-0 loads are dropped by the compiler). The loop runs a fixed number of
            trips per thread, unrolled whole up to 16 (else by 8): a thread past the end evaluates the last
            element again (its loads stay in bounds) and stores that same value to it, so no load sits
            behind a per-trip branch (the compiler would sink it into the guarded store) and every trip's
            loads are in flight together."""
            k.emit(element(k.unflatten(ZERO, shape) if shape else []))
            iterations = -(-count // threads)
            ragged = count % threads != 0

            def trip_header() -> object:
                k.line(f"const uint32_t slot = threadIdx.x + trip * {threads}u;")
                k.line(f"const uint32_t i = slot < {count}u ? slot : {count - 1}u;" if ragged else "const uint32_t i = slot;")
                node = element(k.unflatten(Aff.of(Atom("i", count - 1)), shape) if shape else [])
                return node

            # Whole-unrolled loops of many trips whose loads fit in registers are split in two: every trip's
            # loads first (into per-trip arrays), then, past a scheduling barrier, every trip's arithmetic.
            # In one loop the compiler interleaves later trips' loads with earlier trips' arithmetic and
            # waits for each; a few trips it already requests together.
            # (Loads that do not depend on the trip were emitted with element 0 and are not repeated.)
            arrays: List[str] = []
            split = SPLIT_STAGING_TRIPS <= iterations <= 16
            if split:
                mark, indent = len(k.lines), k.indent
                declarations = []
                k.line("#pragma unroll")
                with k.block(f"for (uint32_t trip = 0; trip < {iterations}u; ++trip) {{"):
                    loads = [load for load in k.load_nodes(trip_header()) if load not in k.nodes]
                    words = sum(2 if is_int(load[2]) else 1 for load in loads)
                    split = 0 < words * iterations <= STAGED_LOAD_REGISTERS
                    for load in loads if split else []:
                        arrays.append(k.fresh("pre"))
                        declarations.append(f"{'int64_t' if is_int(load[2]) else 'float'} {arrays[-1]}[{iterations}];")
                        k.line(f"{arrays[-1]}[trip] = {k.emit(load)};")
                if split:
                    k.lines[mark:mark] = ["    " * indent + line for line in declarations]
                    k.line('__asm__ volatile("" ::: "memory");')
                else:
                    del k.lines[mark:]
            k.line(f"#pragma unroll {iterations if iterations <= 16 else 8}")
            with k.block(f"for (uint32_t trip = 0; trip < {iterations}u; ++trip) {{"):
                node = trip_header()
                if split:
                    loads = [load for load in k.load_nodes(node) if load not in k.nodes]
                    assert len(loads) == len(arrays), "two traversals of one staged element differ"
                    for load, array in zip(loads, arrays):
                        k.nodes[load] = f"{array}[trip]"
                k.line(f"{target}[i] = {k.emit(node)};")

        def stage_rows(value: Value, key: str) -> bool:
            """Evaluate ``value`` once into a __shared__ float array (row-major) read in its place."""
            shape = _shape(value.shape)
            count = math.prod(shape)
            if count > budget[0]:
                return False
            budget[0] -= count
            array = k.fresh("hs")
            k.line(f"__shared__ float {array}[{count}];")
            staging_loop(count, lambda coords: self.read(k, value, coords), shape if value.shape else [], array)
            k.staged_values[key] = array
            return True

        # A buffer computed in place is evaluated once into LDS (every later read in this kernel, and
        # the first workgroup's store of it, come from there) ...
        if any([stage_rows(k.unstored[buffer], buffer) for buffer in resolved]):
            k.line("chroma::lds_barrier();")
        for buffer in resolved:
            expression = k.unstored[buffer]
            shape = _shape(expression.shape)
            count = math.prod(shape)
            slot = k.slot(buffer, expression.dtype, writable=True, extent=self.extents[buffer])
            with k.block("if (blockIdx.x == 0u && blockIdx.y == 0u && blockIdx.z == 0u) {"):
                with k.block(f"for (uint32_t i = threadIdx.x; i < {count}u; i += {threads}u) {{"):
                    i = Aff.of(Atom("i", count - 1))
                    node = ("lds", k.staged_values[buffer], i) if buffer in k.staged_values else self.read(k, expression, k.unflatten(i, shape) if expression.shape else [])
                    k.store(slot, expression.dtype, i, node)
        # ... and so is a deferred norm's operand that still costs loads (it is read twice: squares,
        # then scaling).
        staged_sources = False
        for name in sorted(self.pending_of.get(x.name, frozenset())):
            if name in self.materialized:
                continue
            source = self.pending_norms[name][1]
            if source.name in k.staged_values or (source.stored and source.root.name in k.staged_values):
                continue
            loads = (source.stored and source.root.name in k.unstored) or (
                not source.stored and any(buffer not in k.staged_values for buffer in self.sources[source.name]))
            if loads and stage_rows(source, source.name):
                staged_sources = True
        if staged_sources:
            k.line("chroma::lds_barrier();")
        k.norm_scales = {}
        for name in sorted(self.pending_of.get(x.name, frozenset())):
            if name in self.materialized:
                continue
            _, source, _, epsilon = self.pending_norms[name]
            shape = _shape(source.shape)
            norm_rows, columns = math.prod(shape) // shape[-1], shape[-1]
            scales = k.fresh("ns")
            k.line(f"__shared__ float {scales}[{norm_rows}];")
            # All rows at once: ``lanes`` consecutive threads (a power of two, at most a wave) sum the
            # squares of one row and meet through a butterfly.
            span = 1 << (norm_rows - 1).bit_length()
            lanes = max(1, threads // span)
            with k.block("{"):
                k.line(f"const uint32_t nr = threadIdx.x / {lanes}u, nl = threadIdx.x % {lanes}u;")
                k.line("float squares = 0.0f;")
                with k.block(f"if (nr < {norm_rows}u) {{"):
                    r_atom = Aff.of(Atom("nr", norm_rows - 1))
                    row_coords = k.unflatten(r_atom, shape[:-1]) if len(shape) > 1 else []
                    k.line("#pragma unroll 4")
                    with k.block(f"for (uint32_t c = nl; c < {columns}u; c += {lanes}u) {{"):
                        value = k.emit(self.read(k, source, [*row_coords, Aff.of(Atom("c", columns - 1))]))
                        k.line(f"squares += {value} * {value};")
                k.line(f"for (uint32_t o = {min(lanes, 64) // 2}u; o > 0u; o >>= 1) squares += __shfl_xor(squares, int(o), 64);")
                formula = f"1.0f / sqrtf(total / {float_literal(columns)} + {float_literal(epsilon)})"
                if lanes <= 64:
                    k.line(f"if (nl == 0u && nr < {norm_rows}u) {{ const float total = squares; {scales}[nr] = {formula}; }}")
                else:
                    # a row spans several waves: their sums meet in LDS
                    per_row = lanes // 64
                    k.line(f"__shared__ float {scales}_waves[{threads // 64}];")
                    k.line(f"if (threadIdx.x % 64u == 0u) {scales}_waves[threadIdx.x / 64u] = squares;")
                    k.line("chroma::lds_barrier();")
                    k.line(f"if (nl == 0u && nr < {norm_rows}u) {{ float total = 0.0f; "
                           f"for (uint32_t w = 0; w < {per_row}u; ++w) total += {scales}_waves[nr * {per_row}u + w]; {scales}[nr] = {formula}; }}")
            k.norm_scales[name] = scales
        if k.norm_scales:
            k.line("chroma::lds_barrier();")
        k.line(f"__shared__ float {array}[{rows * inner}];")
        staging_loop(rows * inner, lambda coords: self.read(k, x, [*coords_of(coords[0]), coords[1]]), (rows, inner), array)
        k.line("chroma::lds_barrier();")
        k.norm_scales = {}

    def _norm_kernel(self, meta, x: Value, weight: Value, epsilon: float) -> Value:
        out = self.allocate(tuple(meta.shape), meta.dtype)
        shape = _shape(x.shape)
        columns = shape[-1]
        rows = math.prod(shape) // columns
        dim = len(shape) - 1
        threads, lanes, chunks, resident = self._row_plan(columns, x.dtype)
        splits, chunk, split_lanes = self._row_splits(rows, columns, x.dtype)
        coop = self._coop_plan(rows, columns, x.dtype, "rmsnorm")
        if coop is not None and not resident:
            self._coop_rows("rmsnorm", out, x, shape, dim, columns, rows, coop, weight=weight, epsilon=epsilon)
            self.parallel_reductions += 1
            return out
        if splits > 1 and not resident:
            self._split_norm(out, x, weight, epsilon, shape, rows, columns, splits, chunk, split_lanes)
            self.parallel_reductions += 1
            return out
        k, prologue = self._rmsnorm_rows(out, x, weight, epsilon)
        self.launch(k, rows, threads, [x, weight], kind="rmsnorm", prologue=prologue)
        self.parallel_reductions += 1
        self.last_norm = {"index": len(self.launches) - 1, "args": (out, x, weight, epsilon), "rows": rows, "threads": threads}
        return out

    def _rmsnorm_rows(self, out: Value, x: Value, weight: Value, epsilon: float, epilogue: Optional[Tuple[Value, Value]] = None,
                      store_norm: bool = True) -> Tuple[Kernel, List[str]]:
        """The one-workgroup-per-row RMSNorm kernel writing ``out`` (and its shared-memory prologue). With
        ``epilogue`` = (value, buffer) it also writes ``value``, an elementwise expression of ``out`` (the
        bfloat16 cast the workloads' norm ends with), into ``buffer`` from the normalised lanes it holds,
        and writes ``out`` itself only if ``store_norm``; a read of ``out`` at any other element raises
        ``_NotFusible``."""
        shape = _shape(x.shape)
        columns = shape[-1]
        rows = math.prod(shape) // columns
        dim = len(shape) - 1
        threads, lanes, chunks, resident = self._row_plan(columns, x.dtype)
        waves = threads // 64
        k = Kernel(lanes)
        slot = k.slot(out.name, out.dtype, writable=True, extent=self.extents[out.name]) if store_norm else None
        extra = None if epilogue is None else k.slot(epilogue[1].name, epilogue[1].dtype, writable=True, extent=self.extents[epilogue[1].name])
        row = Aff.of(k.atom("blockIdx.x", rows - 1, prefix="r"))
        step = threads * lanes
        ragged = columns % step != 0
        eps = float_literal(epsilon)

        def coords(j: Aff) -> List[Aff]:
            return self._row_coords(k, row, shape, dim, j)

        def names_of(node) -> List[str]:
            names = k.emit(node)
            return names if isinstance(names, list) else [names] * lanes

        k.line("float squares = 0.0f;")
        if resident:
            k.line(f"float vals[{chunks}][{lanes}];")
        with k.block(f"for (uint32_t c = 0; c < {chunks}u; ++c) {{") if resident else k.block(
            f"for (uint32_t base = threadIdx.x * {lanes}u; base < {columns}u; base += {step}u) {{"
        ):
            j = Aff.of(k.vector_atom(f"c * {step}u + threadIdx.x * {lanes}u" if resident else "base", columns - 1))
            if resident and ragged:
                k.line(f"if ({j.code()} < {columns}u) {{")
                k.indent += 1
            for lane, name in enumerate(names_of(self.read(k, x, coords(j)))):
                if resident:
                    k.line(f"vals[c][{lane}] = {name};")
                k.line(f"squares += {name} * {name};")
            if resident and ragged:
                k.indent -= 1
                k.line("}")
        k.line(f"squares = chroma::block_sum<{waves}>(squares, scratch);")
        k.line(f"const float scale = 1.0f / sqrtf(squares / {float_literal(columns)} + {eps});")
        with k.block(f"for (uint32_t c = 0; c < {chunks}u; ++c) {{") if resident else k.block(
            f"for (uint32_t base = threadIdx.x * {lanes}u; base < {columns}u; base += {step}u) {{"
        ):
            j = Aff.of(k.vector_atom(f"c * {step}u + threadIdx.x * {lanes}u" if resident else "base", columns - 1))
            if ragged and resident:
                k.line(f"if ({j.code()} < {columns}u) {{")
                k.indent += 1
            xs = [f"vals[c][{lane}]" for lane in range(lanes)] if resident else names_of(self.read(k, x, coords(j)))
            ws = names_of(self.read(k, weight, [j]))
            result = self._lane_values(k, [f"{xv} * scale * {wv}" for xv, wv in zip(xs, ws)])
            at = Kernel.flatten(coords(j), shape)
            if store_norm:
                k.store(slot, out.dtype, at, result)
            if epilogue is not None:
                value, buffer = epilogue
                here = at + out.view.offset

                def normalised(address: Aff) -> tuple:
                    if address != here:
                        raise _NotFusible(f"the expression reads {out.name}[{address.code()}], not the element it stores")
                    return result

                k.register_reads[out.root.name] = normalised
                try:
                    k.store(extra, buffer.dtype, at, self.read(k, value, coords(j)))
                finally:
                    del k.register_reads[out.root.name]
            if ragged and resident:
                k.indent -= 1
                k.line("}")
        return k, [f"__shared__ float scratch[{waves}];"]

    def _split_norm(self, out: Value, x: Value, weight: Value, epsilon: float, shape, rows: int, columns: int, splits: int, chunk: int,
                    lanes: int) -> None:
        """RMSNorm of few wide rows: one workgroup per (row, split) sums the squares of its part of the row
        into a scratch float; then each (row, split) workgroup adds its row's partial sums, forms the
        reference's scale 1 / sqrt(sum / D + eps) and writes its part as x * scale * w."""
        dim = len(shape) - 1
        step = ROW_THREADS * lanes
        waves = ROW_THREADS // 64
        partials = self.allocate((rows * splits,), torch.float32)

        def names_of(k: Kernel, value: Value, coords: List[Aff]) -> List[str]:
            names = k.emit(self.read(k, value, coords))
            return names if isinstance(names, list) else [names] * lanes

        def bounds(k: Kernel) -> None:
            k.line(f"const uint32_t begin = blockIdx.x % {splits}u * {chunk}u;")
            k.line(f"const uint32_t end = begin + {chunk}u < {columns}u ? begin + {chunk}u : {columns}u;")
            k.line(f"uint32_t base = begin + threadIdx.x * {lanes}u;")

        k = Kernel(lanes)
        part_slot = k.slot(partials.name, torch.float32, writable=True, extent=self.extents[partials.name])
        row = Aff.of(k.atom(f"blockIdx.x / {splits}u", rows - 1, prefix="r"))
        bounds(k)
        k.line("float squares = 0.0f;")
        with k.block(f"for (; base + {(ROW_UNROLL - 1) * step}u < end; base += {ROW_UNROLL * step}u) {{"):
            loaded = [names_of(k, x, self._row_coords(k, row, shape, dim, Aff.of(k.vector_atom(f"base + {u * step}u", columns - 1))))
                      for u in range(ROW_UNROLL)]
            for names in loaded:
                k.line("squares += " + " + ".join(f"{n} * {n}" for n in names) + ";")
        with k.block(f"for (; base < end; base += {step}u) {{"):
            names = names_of(k, x, self._row_coords(k, row, shape, dim, Aff.of(k.vector_atom("base", columns - 1))))
            k.line("squares += " + " + ".join(f"{n} * {n}" for n in names) + ";")
        k.line(f"squares = chroma::block_sum<{waves}>(squares, scratch);")
        k.line(f"if (threadIdx.x == 0) {part_slot}[blockIdx.x] = squares;")
        self.launch(k, rows * splits, ROW_THREADS, [x], kind="norm_partials", prologue=[f"__shared__ float scratch[{waves}];"])

        k = Kernel(lanes)
        k.streaming = STREAMING_STORES and math.prod(shape) * ITEMSIZE[out.dtype] >= STREAMING_BYTES
        part_slot = k.slot(partials.name, torch.float32, extent=self.extents[partials.name])
        slot = k.slot(out.name, out.dtype, writable=True, extent=self.extents[out.name])
        row_atom = k.atom(f"blockIdx.x / {splits}u", rows - 1, prefix="r")
        row = Aff.of(row_atom)
        k.line("float squares = 0.0f;")
        k.line(f"for (uint32_t s = threadIdx.x; s < {splits}u; s += {ROW_THREADS}u) squares += {part_slot}[{row_atom.name} * {splits}u + s];")
        k.line(f"squares = chroma::block_sum<{waves}>(squares, scratch);")
        k.line(f"const float scale = 1.0f / sqrtf(squares / {float_literal(columns)} + {float_literal(epsilon)});")
        bounds(k)

        def write(j: Aff, names: List[str]) -> None:
            ws = names_of(k, weight, [j])
            result = self._lane_values(k, [f"{xv} * scale * {wv}" for xv, wv in zip(names, ws)])
            k.store(slot, out.dtype, Kernel.flatten(self._row_coords(k, row, shape, dim, j), shape), result)

        with k.block(f"for (; base + {(ROW_UNROLL - 1) * step}u < end; base += {ROW_UNROLL * step}u) {{"):
            js = [Aff.of(k.vector_atom(f"base + {u * step}u", columns - 1)) for u in range(ROW_UNROLL)]
            loaded = [names_of(k, x, self._row_coords(k, row, shape, dim, j)) for j in js]
            for j, names in zip(js, loaded):
                write(j, names)
        with k.block(f"for (; base < end; base += {step}u) {{"):
            j = Aff.of(k.vector_atom("base", columns - 1))
            write(j, names_of(k, x, self._row_coords(k, row, shape, dim, j)))
        self.launch(k, rows * splits, ROW_THREADS, [x, weight, partials], kind="rmsnorm_split",
                    prologue=[f"__shared__ float scratch[{waves}];"])

    # ------------------------------------------------------------------------------ reduction
    def reduction(self, meta, x: Value, axes: Sequence[int], keepdim: bool, mean: bool) -> Value:
        out = self.allocate(tuple(meta.shape), meta.dtype)
        out_shape = _shape(out.shape)
        x_shape = tuple(x.shape)
        reduce_shape = tuple(x_shape[d] for d in axes) or (1,)
        width = math.prod(reduce_shape)
        outputs = math.prod(out_shape)
        parallel = width >= 64
        k = Kernel(1)
        slot = k.slot(out.name, out.dtype, writable=True, extent=self.extents[out.name])
        divisor = float_literal(width if mean else 1)

        def element(out_coords: List[Aff], reduce_coords: List[Aff]) -> tuple:
            coords, o, r = [], 0, 0
            kept = [c for c, size in zip(out_coords, out_shape)] if out.shape else []
            for d in range(len(x_shape)):
                if d in axes:
                    coords.append(reduce_coords[r])
                    r += 1
                    if keepdim:
                        o += 1
                else:
                    coords.append(kept[o])
                    o += 1
            return self.read(k, x, coords)

        if parallel:
            groups = 4
            k.line(f"const uint32_t o = blockIdx.x * {groups}u + threadIdx.x / 64u;")
            k.line(f"if (o >= {outputs}u) return;")
            k.line("float sum = 0.0f;")
            out_coords = k.unflatten(Aff.of(Atom("o", outputs - 1)), out_shape) if out.shape else []
            with k.block(f"for (uint32_t r = threadIdx.x % 64u; r < {width}u; r += 64u) {{"):
                reduce_coords = k.unflatten(Aff.of(Atom("r", width - 1)), reduce_shape)
                k.line(f"sum += {k.emit(element(out_coords, reduce_coords))};")
            k.line("sum = chroma::wave_sum(sum);")
            k.line("if (threadIdx.x % 64u == 0) {")
            k.indent += 1
            k.store(slot, out.dtype, Aff.of(Atom("o", outputs - 1)), self._lane_values(k, [f"sum / {divisor}"]))
            k.indent -= 1
            k.line("}")
            self.launch(k, -(-outputs // groups), 64 * groups, [x], kind="reduce_waves")
            self.parallel_reductions += 1
        else:
            with k.block(f"for (uint32_t o = blockIdx.x * 256u + threadIdx.x; o < {outputs}u; o += gridDim.x * 256u) {{"):
                out_coords = k.unflatten(Aff.of(Atom("o", outputs - 1)), out_shape) if out.shape else []
                k.line("float sum = 0.0f;")
                with k.block(f"for (uint32_t r = 0; r < {width}u; ++r) {{"):
                    reduce_coords = k.unflatten(Aff.of(Atom("r", width - 1)), reduce_shape)
                    k.line(f"sum += {k.emit(element(out_coords, reduce_coords))};")
                k.store(slot, out.dtype, Aff.of(Atom("o", outputs - 1)), self._lane_values(k, [f"sum / {divisor}"]))
            self.launch(k, max(1, min(-(-outputs // 256), MAX_GRID)), 256, [x], kind="reduce")
        return out

    # ------------------------------------------------------------------------------------ top-k
    def topk(self, meta, x: Value, dim: int, largest: bool, sort: bool):
        values = self.allocate(tuple(meta[0].shape), meta[0].dtype)
        indices = self.allocate(tuple(meta[1].shape), meta[1].dtype)
        if self._router(meta, x, dim, largest, sort, values, indices):
            return values, indices
        shape = tuple(x.shape)
        width, inner, outer = self._row_layout(shape, dim)
        count = meta[0].shape[dim]
        rows = outer * inner
        per_lane = -(-width // 64)
        if per_lane > WIDE_TOPK_LANE_VALUES:
            self._wide_topk(meta, x, dim, largest, values, indices)
            return values, indices
        groups = 4
        k = Kernel(1)
        value_slot = k.slot(values.name, values.dtype, writable=True, extent=self.extents[values.name])
        index_slot = k.slot(indices.name, indices.dtype, writable=True, extent=self.extents[indices.name])
        k.line(f"const uint32_t r = blockIdx.x * {groups}u + threadIdx.x / 64u;")
        k.line(f"if (r >= {rows}u) return;")
        k.line("const uint32_t lane = threadIdx.x % 64u;")
        k.line(f"uint64_t keys[{per_lane}];")
        k.line(f"float vals[{per_lane}];")
        row = Aff.of(Atom("r", rows - 1))
        k.line("#pragma unroll")
        with k.block(f"for (uint32_t p = 0; p < {per_lane}u; ++p) {{"):
            k.line("const uint32_t j = p * 64u + lane;")
            k.line(f"if (j < {width}u) {{")
            k.indent += 1
            j = Aff.of(Atom("j", width - 1))
            name = k.emit(self.read(k, x, self._row_coords(k, row, shape, dim, j)))
            k.line(f"vals[p] = {name}; keys[p] = chroma::topk_key({name}, j, {str(bool(largest)).lower()});")
            k.indent -= 1
            k.line("} else { vals[p] = 0.0f; keys[p] = 0; }")
        with k.block(f"for (uint32_t s = 0; s < {count}u; ++s) {{"):
            k.line("uint64_t best = 0;")
            k.line("#pragma unroll")
            k.line(f"for (uint32_t p = 0; p < {per_lane}u; ++p) best = keys[p] > best ? keys[p] : best;")
            k.line("const uint64_t top = chroma::wave_max_u64(best);")
            k.line("const uint32_t winner = 0xffffffffu - uint32_t(top);")
            k.line("if (winner % 64u == lane) {")
            k.indent += 1
            k.line("float chosen = 0.0f;")
            k.line("#pragma unroll")
            k.line(f"for (uint32_t p = 0; p < {per_lane}u; ++p) if (p == winner / 64u) {{ chosen = vals[p]; keys[p] = 0; }}")
            s = Aff.of(Atom("s", count - 1))
            out_coords = self._row_coords(k, row, tuple(meta[0].shape), dim, s)
            address = Kernel.flatten(out_coords, tuple(meta[0].shape))
            k.store(value_slot, values.dtype, address, self._lane_values(k, ["chosen"]))
            k.line(f"{index_slot}[{address.code()}] = int64_t(winner);")
            k.indent -= 1
            k.line("}")
        self.launch(k, -(-rows // groups), 64 * groups, [x], kind="topk")
        return values, indices

    def _router(self, meta, x: Value, dim: int, largest: bool, sort: bool, values: Value, indices: Value) -> bool:
        """Top-k of a few-row linear's output that was the last launch (a mixture-of-experts router): the
        linear launch is replaced by one kernel per row that recomputes its logits (writing them, so any
        other reader of the linear still finds them), selects the top k and also writes the softmax of
        the selected values, which ``softmax`` then returns without a launch."""
        entry = self.retractable.get(x.name)
        if entry is None or entry[0] != len(self.launches) - 1 or not sort or dim != len(x.shape) - 1:
            return False
        _, source, weight, bias, rows, columns, inner = entry
        count = values.shape[dim]
        if x.dtype not in (torch.float32, torch.bfloat16) or math.prod(values.shape) != rows * count:
            return False
        self._retract_last_launch()  # the replacement kernel stages the same operand (and writes its pending stores)
        weights = self.allocate(tuple(values.shape), values.dtype)
        k = Kernel(1)
        per_chunk = 16 // ITEMSIZE[x.dtype]
        chunks = inner // per_chunk if inner % per_chunk == 0 else 0
        lanes = next((l for l in (64, 32, 16, 8, 4, 2) if chunks and chunks % l == 0 and chunks // l >= 4), 1 if chunks else 0)
        if lanes and columns <= 64 and columns * inner * ITEMSIZE[x.dtype] > FUSED_ROUTER_BYTES and chunks // lanes <= 64 and rows <= ROUTER_TICKETS:
            self._split_router(k, source, x, weight, bias, values, indices, weights, rows, columns, inner, lanes, bool(largest), count)
            return True
        row = Aff.of(k.atom("blockIdx.x", rows - 1, prefix="r"))
        lead = tuple(source.shape[:-1])
        ctype = ctype_of(x.dtype)
        w_arg = self._matrix_slot(k, weight)
        self._stage(k, source, 1, inner, lambda _r: k.unflatten(row, lead) if lead else [], 256)
        if lanes:
            # the gate weights are requested after the prologue: vector loads complete in order, so a
            # stream requested first would hold back every dependent load of the prologue behind it
            k.line(f"chroma::StreamStep<{inner}, {lanes}, 1, {ctype}> prefetched;")
            k.line(f"chroma::router_fetch<{columns}>(prefetched, {w_arg});")
        b_arg = self._matrix_slot(k, bias) if bias is not None else "nullptr"
        logits = k.slot(x.name, x.dtype, writable=True, extent=self.extents[x.name])
        value_slot = k.slot(values.name, values.dtype, writable=True, extent=self.extents[values.name])
        index_slot = k.slot(indices.name, indices.dtype, writable=True, extent=self.extents[indices.name])
        weight_slot = k.slot(weights.name, weights.dtype, writable=True, extent=self.extents[weights.name])
        r = row.code()
        k.line(
            f"chroma::router_row<{columns}, {inner}, {lanes}, {str(bool(largest)).lower()}, {ctype}>(xs, {w_arg}, {b_arg}, {logits} + {r} * {columns}u, "
            f"{value_slot} + {r} * {count}u, {index_slot} + {r} * {count}u, {weight_slot} + {r} * {count}u, {count}u"
            + (", prefetched);" if lanes else ");")
        )
        self.launch(k, rows, 256, [source, weight] + ([bias] if bias is not None else []), kind="router")
        self.router_weights[values.name] = weights
        self.router_launches[indices.name] = dict(index=len(self.launches) - 1, source=source, weight=weight, bias=bias, logits=x, values=values,
                                                  indices=indices, weights=weights, rows=rows, columns=columns, inner=inner, lanes=lanes,
                                                  largest=bool(largest), count=count)
        self.fused_routers += 1
        return True

    def _split_router(self, k: Kernel, source: Value, x: Value, weight: Value, bias: Optional[Value], values: Value, indices: Value,
                      weights: Value, rows: int, columns: int, inner: int, lanes: int, largest: bool, count: int) -> None:
        """A router over gate weights too large for one workgroup (``router_split``): parts of 64 / lanes
        experts each per row (4-wave workgroups: all stage the row, the first wave streams the part's gate
        rows), the last part to finish selecting; its per-row ticket counters are
        words of the program's error region (zero at load, returned to zero by every launch)."""
        parts = -(-columns // (64 // lanes))
        row = Aff.of(k.atom("blockIdx.y", rows - 1, prefix="r"))
        lead = tuple(source.shape[:-1])
        ctype = ctype_of(x.dtype)
        w_arg = self._matrix_slot(k, weight)
        b_arg = self._matrix_slot(k, bias) if bias is not None else "nullptr"
        self._stage(k, source, 1, inner, lambda _r: k.unflatten(row, lead) if lead else [], 256)
        outputs = [k.slot(v.name, v.dtype, writable=True, extent=self.extents[v.name]) for v in (x, values, indices, weights)]
        k.uses_error = True
        k.line(
            f"chroma::router_split<{columns}, {inner}, {lanes}, {str(largest).lower()}, {ctype}>(xs, {w_arg}, {b_arg}, {outputs[0]}, "
            f"{outputs[1]}, {outputs[2]}, {outputs[3]}, {count}u, error + chroma::kRouterTicketWord);"
        )
        self.launch(k, (parts, rows, 1), 256, [source, weight] + ([bias] if bias is not None else []), kind="router_split")
        self.router_weights[values.name] = weights
        self.fused_routers += 1

    # =================================================================================== linear
    def linear(self, meta, x: Value, weight: Value, bias: Optional[Value]) -> Value:
        rows, columns, inner = math.prod(x.shape[:-1]), weight.shape[0], weight.shape[1]
        if max(rows, columns, inner) > 2**31 - 1:
            raise ValueError("Matrix dimensions exceed the integer range of the matrix kernels")
        weight = self.contiguous(weight)
        bias = self.contiguous(bias) if bias is not None else None
        out = self.allocate(tuple(meta.shape), meta.dtype)
        dtypes = {x.dtype, weight.dtype, meta.dtype} | ({bias.dtype} if bias is not None else set())
        if len(dtypes) != 1:
            raise NotImplementedError(f"mixed-dtype linear {dtypes}")
        if self.blas and rows <= 16 and self._attention_epilogue(out, x, weight, bias, rows, columns, inner):
            self.skinny_matmuls += 1
            return out
        plan = self._stream_plan(rows, inner, meta.dtype, columns * inner * ITEMSIZE[meta.dtype])
        if (self.blas and rows <= 16 and plan is not None and rows * inner <= LINEAR_STAGED_FLOATS
                and weight.view.offset % (16 // ITEMSIZE[weight.dtype]) == 0):
            self._stream_linear(out, x, weight, bias, rows, columns, inner, plan)
            self.skinny_matmuls += 1
            if columns <= 64:
                self.retractable[out.name] = (len(self.launches) - 1, x, weight, bias, rows, columns, inner)
            return out
        x = self.contiguous(x)
        inputs = [x, weight] + ([bias] if bias is not None else [])
        if self.blas and rows <= 16 and inner % 4 == 0:
            self._skinny_linear(out, x, weight, bias, rows, columns, inner)
            self.skinny_matmuls += 1
        elif (self.blas and columns <= NARROW_COLUMNS and rows >= 64 and inner % (32 if meta.dtype == torch.bfloat16 else 4) == 0
              and x.view.offset % 8 == 0 and weight.view.offset % 8 == 0):
            self._narrow_linear(out, x, weight, bias, rows, columns, inner)
            self.mfma_matmuls += 1
        elif self.blas and inner % (8 if meta.dtype == torch.bfloat16 else 4) == 0:
            self._mfma_linear(out, x, weight, bias, rows, columns, inner)
            self.mfma_matmuls += 1
        elif self.blas:
            self._tiled_linear(out, x, weight, bias, rows, columns, inner)
            self.tiled_matmuls += 1
        else:
            self._scalar_linear(out, x, weight, bias, rows, columns, inner)
        return out

    def _matrix_slot(self, k: Kernel, value: Value) -> str:
        """A pointer to a stored, row-major value (an alias is rebased onto its root at its offset)."""
        root = value.root
        if root.name in k.unstored:
            raise AssertionError(f"{root.name} is computed in place by this kernel and has no stored copy to point at")
        slot = k.slot(root.name, root.dtype)
        offset = value.view.offset
        return f"({slot} + {offset}u)" if offset else slot

    @staticmethod
    def _stream_plan(rows: int, inner: int, dtype: torch.dtype, weight_bytes: int) -> Optional[Tuple[int, int]]:
        """(lanes per row, rows per step) for ``stream_rows``: 64 lanes per row when a row has at least 64
        16-byte chunks, wastes at most 1/8 of its lanes' chunks on a ragged end and the launch stays within
        ``FOLDED_STAGING_BLOCKS`` workgroups (or the narrower layout would exceed them too); otherwise the
        widest power-of-two lane group that gives each lane 4 or more whole chunks (or a whole short row).
        Products streaming at most ``SPREAD_BYTES`` of
        weights take one row step per wave; larger ones take more only as far as needed to stay within
        ``FOLDED_STAGING_BLOCKS`` workgroups (up to ~32 chunks per lane in flight). A workgroup's stream is
        bounded by its compute unit's outstanding requests, so products go fastest spread over as many
        compute units as they have rows for. None when a row is not a whole number of chunks."""
        per_chunk = 16 // ITEMSIZE[dtype]
        if inner % per_chunk:
            return None
        chunks = inner // per_chunk
        rows_of_w = weight_bytes // (inner * ITEMSIZE[dtype])

        def plan(lanes: int) -> Optional[Tuple[int, int, int]]:
            per_lane = -(-chunks // lanes)
            if per_lane > 64:
                return None
            if weight_bytes <= SPREAD_BYTES:
                return lanes, 1, 0
            # Up to ~32 chunks per lane in flight, but more row steps per wave only while the launch would
            # otherwise exceed FOLDED_STAGING_BLOCKS workgroups: more workgroups stream faster than more rows
            # per wave (a workgroup's stream is bounded by its compute unit's outstanding requests).
            most = max(1, min(8, 32 // per_lane, max(1, 32 // rows)))
            steps = 1
            while steps < most and -(-rows_of_w // (64 // lanes * steps * 4)) > FOLDED_STAGING_BLOCKS:
                steps += 1
            if rows > 1 and -(-rows_of_w // (64 // lanes * steps * 4)) > FOLDED_STAGING_BLOCKS:
                # out of reach: a product of several X rows then streams fastest one row step per wave over
                # the most workgroups (C3's 8-row vocabulary product, 8 x 4 -> 8 x 1: forward 335.8 -> 318.7 us)
                steps = 1
            return lanes, steps, -(-rows_of_w // (64 // lanes * steps * 4))

        wide = -(-chunks // 64)
        whole_rows = None
        if chunks >= 64 and (wide * 64 - chunks) * 8 <= wide * 64:
            # 64 lanes per row (a ragged last chunk costs at most 1/8 of a lane's chunks): a wave covers one
            # row per step, so the product spreads over as many workgroups as its rows allow
            whole_rows = plan(64)
            if whole_rows is not None and whole_rows[2] <= FOLDED_STAGING_BLOCKS:
                return whole_rows[0], whole_rows[1]
        lanes = next((l for l in (64, 32, 16, 8, 4, 2) if chunks % l == 0 and chunks // l >= 4), 1)
        chosen = plan(lanes)
        if whole_rows is not None and (chosen is None or chosen[2] > FOLDED_STAGING_BLOCKS):
            # neither stays within FOLDED_STAGING_BLOCKS (a vocabulary-sized W): whole rows per load, 1 KiB
            # of one row per wave instruction, stream faster than 8 rows x 128 B (GPT-OSS-20B unembedding,
            # 1.16 GB: the decode step 40 us shorter)
            return whole_rows[0], whole_rows[1]
        return None if chosen is None else (chosen[0], chosen[1])

    def _stream_blocks(self, columns: int, lanes: int, steps: int) -> int:
        waves = -(-columns // (64 // lanes * steps))
        return max(1, min(-(-waves // 4), STREAM_BLOCKS))

    def _stream_linear(self, out, x, weight, bias, rows, columns, inner, plan) -> None:
        """A few-row linear on the weight-streaming kernel; X (any view or fused expression, including a
        deferred norm) is evaluated into LDS by the generated prologue."""
        lanes, steps = plan
        blocks, threads = self._stream_blocks(columns, lanes, steps), 256
        x = self._stageable(x, blocks)
        k = Kernel(1)
        w_arg = self._matrix_slot(k, weight)
        b_arg = self._matrix_slot(k, bias) if bias is not None else "nullptr"
        out_slot = k.slot(out.name, out.dtype, writable=True, extent=self.extents[out.name])
        lead = tuple(x.shape[:-1])
        # A large W is requested after the prologue that stages X: vector loads complete in order, so a
        # stream requested first makes every dependent load of the prologue wait for it (and queue behind
        # it); measured on the GPT-OSS-20B decode products, the prologue then costs several times its own
        # latency. A small W (a few KiB per workgroup) arrives while the prologue runs, so it goes first.
        early = columns * inner * ITEMSIZE[weight.dtype] <= EARLY_FETCH_BYTES
        fetch = [f"chroma::StreamStep<{inner}, {lanes}, {steps}, {ctype_of(out.dtype)}> prefetched;",
                 f"chroma::stream_linear_fetch(prefetched, {w_arg}, {columns}u);"]
        if early:
            for line in fetch:
                k.line(line)
        self._stage(k, x, rows, inner, lambda row: k.unflatten(row, lead) if lead else [], threads)
        if not early:
            for line in fetch:
                k.line(line)
        k.line(
            f"chroma::stream_linear<{rows}, {inner}, {lanes}, {steps}, true, {ctype_of(out.dtype)}>("
            f"nullptr, xs, {w_arg}, {b_arg}, {out_slot}, {columns}u, prefetched);"
        )
        self.launch(k, blocks, threads, [x, weight] + ([bias] if bias is not None else []), kind="linear_stream")

    def _narrow_linear(self, out, x, weight, bias, rows, columns, inner) -> None:
        """Many rows, few columns (a router's gate over a prefill): ``narrow_linear``, one workgroup per 16
        rows, instead of 128 x 128 tiles that would leave all but a few compute units idle."""
        k = Kernel(1)
        args = [self._matrix_slot(k, x), self._matrix_slot(k, weight), self._matrix_slot(k, bias) if bias is not None else "nullptr"]
        out_slot = k.slot(out.name, out.dtype, writable=True, extent=self.extents[out.name])
        k.line(f"chroma::narrow_linear<{ctype_of(out.dtype)}, {columns}>({args[0]}, {args[1]}, {args[2]}, {out_slot}, {rows}u, {inner}u);")
        self.launch(k, -(-rows // 16), 256, [x, weight] + ([bias] if bias is not None else []), kind="linear_narrow")

    def _skinny_linear(self, out, x, weight, bias, rows, columns, inner) -> None:
        lanes_per_row = 64
        while lanes_per_row > 1 and inner % (4 * lanes_per_row):
            lanes_per_row //= 2
        k = Kernel(1)
        args = [self._matrix_slot(k, x), self._matrix_slot(k, weight), self._matrix_slot(k, bias) if bias is not None else "nullptr"]
        out_slot = k.slot(out.name, out.dtype, writable=True, extent=self.extents[out.name])
        rows_per_wave = 64 // lanes_per_row
        waves = -(-columns // rows_per_wave)
        blocks = min(-(-waves // 4), 8192)
        ctype = ctype_of(out.dtype)
        k.line(
            f"chroma::skinny_linear<{rows}, {inner}, {lanes_per_row}, {ctype}>("
            f"{args[0]}, {args[1]}, {args[2]}, {out_slot}, {columns}u);"
        )
        self.launch(k, blocks, 256, [x, weight] + ([bias] if bias is not None else []), kind="linear_skinny")

    def _prefetch_weight(self, weight: Value) -> None:
        """Launch ``prefetch_bytes`` over a constant weight of PREFETCH_WEIGHT_BYTES (see there)."""
        size = math.prod(weight.shape) * ITEMSIZE[weight.dtype]
        offset = weight.view.offset * ITEMSIZE[weight.dtype] if weight.view is not None else 0
        low, high = PREFETCH_WEIGHT_BYTES
        if (not WEIGHT_PREFETCH or not low <= size <= high or offset % 16 or not weight.stored
                or self.binding_of(weight.root.name).kind != "weight"):
            return
        k = Kernel(1)
        k.line(f"chroma::prefetch_bytes({self._matrix_slot(k, weight)}, {size - size % 16}ull);")
        self.launch(k, min(-(-size // (16 * 256)), PREFETCH_BLOCKS), 256, [weight], kind="prefetch")
        self.weight_prefetches += 1

    def _mfma_linear(self, out, x, weight, bias, rows, columns, inner) -> None:
        if not self._wide_gemm(out.dtype, inner, rows, columns):
            # (the wide body's C5 QKV product gains 3.4 us from warm weights, less than the 6.6 us read-ahead;
            # the mid body's output projection 15 us for 5.5)
            self._prefetch_weight(weight)
        k = Kernel(1)
        args = [self._matrix_slot(k, x), self._matrix_slot(k, weight), self._matrix_slot(k, bias) if bias is not None else "nullptr"]
        out_slot = k.slot(out.name, out.dtype, writable=True, extent=self.extents[out.name])
        tiles = -(-columns // 128) * -(-rows // 128)
        # the 64-deep body (two workgroups per CU) when every tile fits in one round of the chip, else the
        # 32-deep body (three per CU), whose rounds quantize less
        path = 0 if tiles <= 2 * MFMA_CUS else 1
        threads = 256
        if self._wide_gemm(out.dtype, inner, rows, columns):
            wide_tiles = -(-rows // WIDE_GEMM_TILE[0]) * -(-columns // WIDE_GEMM_TILE[1])
            k.min_waves = 1
            k.line(f"chroma::mfma_linear_wide<{ctype_of(out.dtype)}>({args[0]}, {args[1]}, {args[2]}, {out_slot}, {rows}u, {columns}u, {inner}u);")
            self.launch(k, 8 * -(-wide_tiles // 8), WIDE_GEMM_THREADS, [x, weight] + ([bias] if bias is not None else []), kind="linear_wide")
            return
        mid_tiles = -(-rows // MID_GEMM_TILE[0]) * -(-columns // MID_GEMM_TILE[1])
        if MID_GEMMS and out.dtype == torch.bfloat16 and inner % 32 == 0 and mid_tiles >= MID_GEMM_MIN_TILES:
            k.min_waves = 1
            k.line(f"chroma::mfma_linear_mid<{ctype_of(out.dtype)}>({args[0]}, {args[1]}, {args[2]}, {out_slot}, {rows}u, {columns}u, {inner}u);")
            self.launch(k, 8 * -(-mid_tiles // 8), MID_GEMM_THREADS, [x, weight] + ([bias] if bias is not None else []), kind="linear_mid")
            return
        if self._direct_gemm(out.dtype, inner):
            path, threads = 2, DIRECT_GEMM_THREADS
            k.min_waves = DIRECT_GEMM_BLOCKS
        k.line(f"chroma::mfma_linear<{ctype_of(out.dtype)}, {path}>({args[0]}, {args[1]}, {args[2]}, {out_slot}, {rows}u, {columns}u, {inner}u);")
        self.launch(k, 8 * -(-tiles // 8), threads, [x, weight] + ([bias] if bias is not None else []), kind="linear_mfma")

    @staticmethod
    def _wide_gemm(dtype: torch.dtype, inner: int, rows: int, columns: int) -> bool:
        """The wide matrix-core body (``mfma_gemm_wide``) applies: bfloat16 operands whose contiguous rows
        of ``inner`` elements split into 32-deep slices of 16-byte chunks, in a product large enough to give
        it ``WIDE_GEMM_MIN_TILES`` tiles."""
        tiles = -(-rows // WIDE_GEMM_TILE[0]) * -(-columns // WIDE_GEMM_TILE[1])
        return dtype == torch.bfloat16 and inner % 32 == 0 and tiles >= WIDE_GEMM_MIN_TILES

    @staticmethod
    def _direct_gemm(dtype: torch.dtype, inner: int) -> bool:
        """The direct-to-LDS matrix-core body (``mfma_gemm_direct``) applies: bfloat16 operands whose
        contiguous rows of ``inner`` elements split into 64-deep slices of 16-byte chunks."""
        return dtype == torch.bfloat16 and inner % 64 == 0

    def _tiled_linear(self, out, x, weight, bias, rows, columns, inner) -> None:
        k = Kernel(1)
        args = [self._matrix_slot(k, x), self._matrix_slot(k, weight), self._matrix_slot(k, bias) if bias is not None else "nullptr"]
        out_slot = k.slot(out.name, out.dtype, writable=True, extent=self.extents[out.name])
        ctype = ctype_of(out.dtype)
        k.line(f"chroma::tiled_linear<{ctype}>({args[0]}, {args[1]}, {args[2]}, {out_slot}, {rows}u, {columns}u, {inner}u);")
        self.launch(k, (-(-columns // 64), -(-rows // 64), 1), 256, [x, weight] + ([bias] if bias is not None else []), kind="linear_tiled")

    def _scalar_linear(self, out, x, weight, bias, rows, columns, inner) -> None:
        k = Kernel(1)
        slot = k.slot(out.name, out.dtype, writable=True, extent=self.extents[out.name])
        total = rows * columns
        with k.block(f"for (uint32_t o = blockIdx.x * 256u + threadIdx.x; o < {total}u; o += gridDim.x * 256u) {{"):
            o = Atom("o", total - 1)
            row, column = k.div(Aff.of(o), columns), k.mod(Aff.of(o), columns)
            kk = Aff.of(Atom("kk", inner - 1))
            k.line("float sum = 0.0f;")
            with k.block(f"for (uint32_t kk = 0; kk < {inner}u; ++kk) {{"):
                a = k.emit(self.read_flat(k, x, row.scale(inner) + kk))
                b = k.emit(self.read_flat(k, weight, column.scale(inner) + kk))
                k.line(f"sum += {a} * {b};")
            if bias is not None:
                k.line(f"sum += {k.emit(self.read(k, bias, [column]))};")
            k.store(slot, out.dtype, Aff.of(o), self._lane_values(k, ["sum"]))
        self.launch(k, max(1, min(-(-total // 256), MAX_GRID)), 256, [x, weight] + ([bias] if bias is not None else []), kind="linear_scalar")

    # ============================================================================== attention
    def attention(self, meta, q: Value, k_past: Optional[Value], k_new: Value, v_past: Optional[Value], v_new: Value,
                  mask: Value, sinks: Value, scale: float) -> Value:
        """Grouped-query attention with sinks in one launch (the ``_attention`` node that the graph pass
        substitutes for einsum / scale / mask / cat / softmax / slice / einsum): one workgroup per (query
        row, key-value head), operands read through generated loaders, so views and fused expressions
        (the rotary embedding of q and of the new keys) are evaluated in place."""
        tokens, kv_heads, group, dim = q.shape
        past = k_past.shape[0] if k_past is not None else 0
        keys = past + k_new.shape[0]
        out = self.allocate(tuple(meta.shape), meta.dtype)
        bf16 = meta.dtype == torch.bfloat16
        if self.blas and bf16 and dim % 32 == 0 and dim <= 128 and tokens >= MATRIX_ATTENTION_TOKENS:
            if self._matrix_attention(out, q, k_past, k_new, v_past, v_new, mask, sinks, scale):
                return out
        inputs = [v for v in (q, k_past, k_new, v_past, v_new, mask, sinks) if v is not None]
        rows = self._decode_rows(k_past, v_past, keys - past, dim)
        if rows is not None and keys > 4 * DECODE_SPLIT_KEYS and tokens * kv_heads <= min(63, ATTENTION_TICKETS):
            self._decode_attention(out, q, k_past, k_new, v_past, v_new, mask, sinks, scale, rows, inputs)
            self.fused_attentions += 1
            return out
        splits = -(-keys // SPLIT_KEYS) if keys > 4 * SPLIT_KEYS and tokens * kv_heads < 64 else 1
        if splits == 1 and keys <= WAVE_ATTENTION_KEYS and dim <= 64 and group <= 16:
            # Short key ranges: one wave per query head, wave-level reductions only.
            operands = (out, q, k_past, k_new, v_past, v_new, mask, sinks, scale)
            k = self._waves_attention(*operands)
            self.launch(k, (tokens, kv_heads, 1), 64 * group, inputs, kind="attention")
            if kv_heads == 1:
                # a following few-row linear of the whole row may become this kernel's epilogue
                self.retractable_attention[out.name] = (len(self.launches) - 1, operands, inputs)
        elif splits == 1:
            k, split, _ = self._attention_kernel(out, q, k_past, k_new, v_past, v_new, mask, sinks, None)
            k.line(f"chroma::attention_rows<0, {dim}, {group}, 256, {str(bf16).lower()}>(0u, {keys}u, {float_literal(scale)}, "
                   "load_q, load_k, load_v, load_mask, load_sink, store, chroma::AttentionSplit{nullptr, nullptr, 1u, 0u});")
            self.launch(k, (tokens, kv_heads, 1), 256, inputs, kind="attention")
        else:
            # Long key ranges with few (query, head) rows: the keys are split over workgroups (statistics,
            # then partial p . v with the row's statistics, then the in-order sum of the splits).
            stats = self.allocate((tokens * kv_heads * splits * group * 2,), torch.float32)
            partial = self.allocate((tokens * kv_heads * splits * group * dim,), torch.float32)
            for phase in (1, 2):
                k, split, _ = self._attention_kernel(out, q, k_past, k_new, v_past, v_new, mask, sinks, (stats, partial, splits))
                k.line(f"const uint32_t begin = blockIdx.z * {SPLIT_KEYS}u;")
                k.line(f"const uint32_t end = begin + {SPLIT_KEYS}u < {keys}u ? begin + {SPLIT_KEYS}u : {keys}u;")
                k.line(f"chroma::attention_rows<{phase}, {dim}, {group}, 256, {str(bf16).lower()}>(begin, end, {float_literal(scale)}, "
                       f"load_q, load_k, load_v, load_mask, load_sink, store, {split});")
                self.launch(k, (tokens, kv_heads, splits), 256, inputs + [stats] + ([partial] if phase == 2 else []), kind=f"attention_split{phase}")
            k, _, row = self._attention_kernel(out, q, k_past, k_new, v_past, v_new, mask, sinks, (stats, partial, splits), loaders=False)
            table = k.slot(partial.name, torch.float32, extent=self.extents[partial.name])
            k.line(f"chroma::attention_combine<{dim}, {group}>({table} + {row} * {group * dim}u, {splits}u, store);")
            self.launch(k, (tokens, kv_heads, 1), 256, [partial], kind="attention_combine")
        self.fused_attentions += 1
        return out

    def _waves_attention(self, out, q, k_past, k_new, v_past, v_new, mask, sinks, scale, epilogue=None) -> Kernel:
        """The one-wave-per-query-head attention kernel. ``epilogue`` = (weight, bias, linear output, lanes,
        steps): the workgroup also multiplies its finished row (all heads, rounded as stored) by W^T from
        LDS (W requested before the attention when small, else once it is done)."""
        tokens, kv_heads, group, dim = q.shape
        keys = (k_past.shape[0] if k_past is not None else 0) + k_new.shape[0]
        bf16 = out.dtype == torch.bfloat16
        prelude: List = []
        store_extra: List[str] = []
        if epilogue is not None:
            weight, bias, linear_out, lanes, steps = epilogue
            ctype, inner, columns = ctype_of(out.dtype), group * dim, weight.shape[0]
            prelude.append(lambda k: f"__shared__ float attention_row[{inner}];")
            store_extra = [f"attention_row[g * {dim}u + d] = chroma::storage_round<{str(bf16).lower()}>(value);"]
        k, _, _ = self._attention_kernel(out, q, k_past, k_new, v_past, v_new, mask, sinks, None, prelude=prelude, store_extra=store_extra)
        # A small W is requested before the attention, so its round trip overlaps the attention's own loads;
        # a large one once the attention is done (loads complete in order, see _stream_linear)
        early = epilogue is not None and columns * inner * ITEMSIZE[weight.dtype] <= EARLY_FETCH_BYTES
        fetch = []
        if epilogue is not None:
            fetch = [f"chroma::StreamStep<{inner}, {lanes}, {steps}, {ctype}> prefetched;",
                     f"chroma::stream_block_fetch(prefetched, {self._matrix_slot(k, weight)}, {columns}u);"]
        if early:
            for line in fetch:
                k.line(line)
        k.line(f"chroma::attention_waves<{dim}, {group}, {str(bf16).lower()}>({keys}u, {float_literal(scale)}, "
               "load_q, load_k, load_v, load_mask, load_sink, store);")
        if epilogue is not None:
            b_arg = self._matrix_slot(k, bias) if bias is not None else "nullptr"
            out_slot = k.slot(linear_out.name, linear_out.dtype, writable=True, extent=self.extents[linear_out.name])
            k.line("__syncthreads();")
            if not early:
                for line in fetch:
                    k.line(line)
            k.line(f"chroma::stream_block_linear<1, {inner}, {lanes}, {steps}, true, {ctype}>(nullptr, attention_row, "
                   f"{self._matrix_slot(k, weight)}, {b_arg}, {out_slot} + size_t(blockIdx.x) * {columns}u, {columns}u, prefetched);")
        return k

    def _attention_epilogue(self, out: Value, x: Value, weight: Value, bias: Optional[Value], rows: int, columns: int, inner: int) -> bool:
        """A few-row linear whose X is exactly the rows of the last launch's wave attention (one workgroup
        per query row holding every head): the attention launch is replaced by one that also computes this
        product as its epilogue. False (nothing changed) otherwise."""
        if not x.stored or x.view is None:
            return False
        entry = self.retractable_attention.get(x.root.name)
        if entry is None or entry[0] != len(self.launches) - 1:
            return False
        index, operands, inputs = entry
        attention_out, q = operands[0], operands[1]
        tokens, _, group, dim = q.shape
        natural = contiguous_strides(x.shape)
        if (x.view.offset or rows != tokens or inner != group * dim or x.dtype not in (torch.float32, torch.bfloat16)
                or any(size != 1 and a != b for size, a, b in zip(x.shape, x.view.strides, natural))):
            return False
        per_chunk = 16 // ITEMSIZE[x.dtype]
        if inner % per_chunk or weight.view.offset % per_chunk:
            return False
        chunks = inner // per_chunk
        lanes = next((l for l in (64, 32, 16, 8, 4, 2) if chunks % l == 0 and chunks // l >= 4), 1)
        per_lane = chunks // lanes
        if per_lane > 16:
            return False
        # W split over grid.z parts of about 16 KiB each (one workgroup streams only ~15 GB/s), as far as
        # every part keeps rows at this lane layout; each part recomputes the (few-key) attention row
        rows_per_step = 64 // lanes  # rows of W one wave covers per step
        parts = max(1, min(-(-columns * inner * ITEMSIZE[x.dtype] // (16 << 10)), -(-columns // (rows_per_step * group)), 8))
        # rows of W per wave step: enough to cover W in one step, at most 16 chunks per lane held
        steps = max(1, min(16 // per_lane, -(-columns // (rows_per_step * group * parts))))
        self._retract_last_launch()
        k = self._waves_attention(*operands, epilogue=(weight, bias, out, lanes, steps))
        self.launch(k, (tokens, 1, parts), 64 * group, inputs + [weight] + ([bias] if bias is not None else []), kind="attention_linear")
        self.retractable_attention.pop(x.root.name, None)
        self.attention_epilogues += 1
        return True

    def _retract_last_launch(self) -> Launch:
        """Remove the last launch (its kernel source too when nothing else launches it); the write-through
        stores it performed become pending again."""
        popped = self.launches.pop()
        self.kernels -= 1
        for buffer in self.resolved_by_launch.pop(len(self.launches), []):
            self.pending_stores.add(buffer)
        if all(launch.kernel != popped.kernel for launch in self.launches):
            text = next(src for src, name in self.kernel_names.items() if name == popped.kernel)
            del self.kernel_names[text]
            self.kernel_sources = [text for text in self.kernel_sources if f" {popped.kernel}(" not in text]
        return popped

    def _decode_rows(self, k_past: Optional[Value], v_past: Optional[Value], fresh: int, dim: int) -> Optional[dict]:
        """The in-place layout of the stored key/value rows for ``attention_decode``: {"k"/"v": (stored
        value, element strides, element offset)} when both are stored (or strided views) with contiguous
        head dimensions, 16-byte aligned rows and whole 16-byte chunks per lane group, and the new rows fit
        the LDS staging; else None."""
        if k_past is None or v_past is None or k_past.dtype != v_past.dtype or fresh * dim > STAGED_ROWS:
            return None
        per_chunk = 16 // ITEMSIZE[k_past.dtype]
        lanes = dim // per_chunk
        if dim % per_chunk or lanes > 64 or lanes & (lanes - 1):
            return None
        if -(-DECODE_SPLIT_KEYS // (4 * (64 // lanes))) > 8:
            return None  # a thread would hold more than 8 keys of a split (attention_decode's registers)
        layout = {}
        for name, value in (("k", k_past), ("v", v_past)):
            stored, strides = self._in_place(value)
            if stored is None:
                return None
            strides = [0 if size == 1 else stride for size, stride in zip(value.shape, strides)]
            offset = stored.view.offset if stored.view.base is not None else 0
            if strides[2] not in (0, 1) or value.shape[2] != dim or any(x % per_chunk for x in (*strides[:2], offset)):
                return None
            layout[name] = (stored, strides, offset)
        return layout

    def _decode_attention(self, out, q, k_past, k_new, v_past, v_new, mask, sinks, scale, rows: dict, inputs: List[Value]) -> None:
        """Long key ranges for a few query rows (decode steps) with ``attention_decode``: the keys are split
        over workgroups of ``DECODE_SPLIT_KEYS``; phase 1 writes the masked scores and each split's
        statistics, phase 2 the split's partial p . v sums, and its last split to finish adds the splits in
        order (a ticket per (query row, head) in the program's error region, returned to zero)."""
        tokens, kv_heads, group, dim = q.shape
        past = k_past.shape[0]
        keys = past + k_new.shape[0]
        bf16 = out.dtype == torch.bfloat16
        splits = -(-keys // DECODE_SPLIT_KEYS)
        stats = self.allocate((tokens * kv_heads * splits * group * 2,), torch.float32)
        partial = self.allocate((tokens * kv_heads * splits * group * dim,), torch.float32)
        scores = self.allocate((tokens * kv_heads * keys * group,), torch.float32)
        ctype = ctype_of(k_past.dtype)
        prelude = [f"const uint32_t begin = blockIdx.z * {DECODE_SPLIT_KEYS}u;",
                   f"const uint32_t end = begin + {DECODE_SPLIT_KEYS}u < {keys}u ? begin + {DECODE_SPLIT_KEYS}u : {keys}u;"]
        for phase in (1, 2):
            # phase 1 reads keys, phase 2 values; only the split that holds the new rows stages them
            needed = "k" if phase == 1 else "v"
            k, split, _ = self._attention_kernel(out, q, k_past, k_new, v_past, v_new, mask, sinks, (stats, partial, splits),
                                                 prelude=prelude, fresh=((f"load_{needed}",), f"end > {past}u"))
            scores_slot = k.slot(scores.name, torch.float32, writable=True, extent=self.extents[scores.name])
            sources = []
            for name in ("k", "v"):
                stored, strides, offset = rows[name]
                root = stored.root
                base = k.slot(root.name, root.dtype, extent=self.extents[root.name])
                staged_rows = f"load_{name}_new" if name == needed else "nullptr"
                sources.append(f"chroma::KeyRows<{ctype}>{{{base} + {offset}u + blockIdx.y * {strides[1]}u, {strides[0]}u, {past}u, {staged_rows}}}")
            k.uses_error = True  # phase 2's last split takes its ticket from the error region
            k.line(f"chroma::attention_decode<{phase}, {dim}, {group}, {str(bf16).lower()}, {ctype}, {DECODE_SPLIT_KEYS}>(begin, end, {float_literal(scale)}, "
                   f"load_q, {sources[0]}, {sources[1]}, load_mask, load_sink, {split}, "
                   f"{scores_slot} + (size_t(blockIdx.x) * {kv_heads}u + blockIdx.y) * {keys * group}u, store, "
                   f"error + chroma::kAttentionTicketWord + blockIdx.x * {kv_heads}u + blockIdx.y);")
            self.launch(k, (tokens, kv_heads, splits), 256, inputs + [stats, scores] + ([partial] if phase == 2 else []), kind=f"attention_decode{phase}")

    def _attention_kernel(self, out, q, k_past, k_new, v_past, v_new, mask, sinks, split, loaders: bool = True,
                          prelude: Sequence = (), fresh: Optional[Tuple[Tuple[str, ...], str]] = None,
                          store_extra: Sequence[str] = ()) -> Tuple[Kernel, str, str]:
        """A kernel over (query row, key/value head) with the attention loaders and the result store
        declared as lambdas (operands read through generated code, so views and fused expressions are
        evaluated in place); returns it with the C expression of its ``AttentionSplit`` and the C
        expression of its first split row in the split scratch. ``prelude`` lines open the kernel;
        ``fresh`` = (key sources, C condition) stages only those sources' new rows, and only in workgroups
        where the condition holds (no ``load_k``/``load_v`` lambdas are declared then)."""
        tokens, kv_heads, group, dim = q.shape
        past = k_past.shape[0] if k_past is not None else 0
        keys = past + k_new.shape[0]
        k = Kernel(1)
        t = Aff.of(k.atom("blockIdx.x", tokens - 1, prefix="t"))
        h = Aff.of(k.atom("blockIdx.y", kv_heads - 1, prefix="h"))
        for line in prelude:
            k.line(line(k) if callable(line) else line)
        slot = k.slot(out.name, out.dtype, writable=True, extent=self.extents[out.name])
        scores_shape = (kv_heads, group, tokens, keys)

        def loader(name: str, params: Sequence[Tuple[str, int]], body: Callable[[List[Aff]], Optional[tuple]], split=None) -> None:
            signature = ", ".join(f"uint32_t {p}" for p, _ in params)
            with k.block(f"auto {name} = [&]({signature}) -> float {{", "};"):
                coords = [Aff.of(Atom(p, hi)) for p, hi in params]
                if split is None:
                    node = body(coords)
                    k.hoist_loads(node)
                    k.line(f"return {k.emit(node)};")
                    return
                bound, first, second = split
                with k.block(f"if ({params[0][0]} < {bound}u) {{"):
                    node = first(coords)
                    k.hoist_loads(node)
                    k.line(f"return {k.emit(node)};")
                node = second(coords)
                k.hoist_loads(node)
                k.line(f"return {k.emit(node)};")

        fresh_only = fresh
        fresh = keys - past
        staged = loaders and fresh * dim <= STAGED_ROWS
        assert fresh_only is None or staged, "selective staging needs the new rows in LDS"

        def key_source(past_value: Optional[Value], new_value: Value, name: str) -> None:
            params = [("j", keys - 1), ("d", dim - 1)]
            if fresh_only is not None and name not in fresh_only[0]:
                return
            if staged:
                # The new rows (often a fused expression such as the rotary embedding) are evaluated once,
                # cooperatively, into LDS; the key loops then read plain LDS values.
                k.line(f"__shared__ float {name}_new[{fresh * dim}];")
                with k.block(f"if ({fresh_only[1]}) {{" if fresh_only is not None else "{"):
                    # Runs of 32 elements, one per wave (its other 32 lanes idle): with head dimensions of 64
                    # or more, each half of a head's row (the two sides of a rotary embedding) is evaluated
                    # by whole waves, without diverging.
                    runs = -(-fresh * dim // 32)
                    with k.block(f"for (uint32_t slot = threadIdx.x; slot < {runs * 64}u; slot += blockDim.x) {{"):
                        k.line("const uint32_t i = slot / 64u * 32u + slot % 64u;")
                        with k.block(f"if (slot % 64u < 32u && i < {fresh * dim}u) {{"):
                            i = Aff.of(Atom("i", fresh * dim - 1))
                            row, column = k.div(i, dim), k.mod(i, dim)
                            node = self.read(k, new_value, [row, h, column])
                            k.hoist_loads(node)
                            k.line(f"{name}_new[i] = {k.emit(node)};")
                if fresh_only is not None:
                    return

            if past_value is None:
                if staged:
                    with k.block(f"auto {name} = [&](uint32_t j, uint32_t d) -> float {{", "};"):
                        k.line(f"return {name}_new[j * {dim}u + d];")
                    return
                loader(name, params, lambda c: self.read(k, new_value, [c[0], h, c[1]]))
                return

            def first(c):
                return self.read(k, past_value, [Aff.of(Atom("j", past - 1)), h, c[1]])

            if staged:
                with k.block(f"auto {name} = [&](uint32_t j, uint32_t d) -> float {{", "};"):
                    with k.block(f"if (j < {past}u) {{"):
                        k.line(f"return {k.emit(first([Aff.of(Atom('j', keys - 1)), Aff.of(Atom('d', dim - 1))]))};")
                    k.line(f"return {name}_new[(j - {past}u) * {dim}u + d];")
                return

            def second(c):
                shifted = k.derived(c[0], f"({{}}) - {past}u", keys - past - 1)
                return self.read(k, new_value, [shifted, h, c[1]])

            loader(name, params, None, split=(past, first, second))

        if loaders:
            loader("load_q", [("g", group - 1), ("d", dim - 1)], lambda c: self.read(k, q, [t, h, c[0], c[1]]))
            key_source(k_past, k_new, "load_k")
            key_source(v_past, v_new, "load_v")
            loader("load_mask", [("j", keys - 1), ("g", group - 1)], lambda c: self.broadcast_read(k, mask, [h, c[1], t, c[0]], scores_shape))
            loader("load_sink", [("g", group - 1)], lambda c: self.broadcast_read(k, sinks, [h, c[0], t, ZERO], scores_shape[:3] + (1,)))
        with k.block("auto store = [&](uint32_t g, uint32_t d, float value) {", "};"):
            g_atom, d_atom = Aff.of(Atom("g", group - 1)), Aff.of(Atom("d", dim - 1))
            node = self._lane_values(k, ["value"])
            k.store(slot, out.dtype, Kernel.flatten([t, h, g_atom, d_atom], out.shape), node)
            for line in store_extra:
                k.line(line)
        if split is None:
            return k, "", ""
        stats, partial, splits = split
        row = f"(size_t({t.code()}) * {kv_heads}u + {h.code()}) * {splits}u"
        stats_slot = k.slot(stats.name, torch.float32, writable=True, extent=self.extents[stats.name]) if loaders else None
        partial_slot = k.slot(partial.name, torch.float32, writable=True, extent=self.extents[partial.name]) if loaders else None
        descriptor = (f"chroma::AttentionSplit{{{stats_slot} + {row} * {group * 2}u, {partial_slot} + {row} * {group * dim}u, "
                      f"{splits}u, blockIdx.z}}") if loaders else ""
        return k, descriptor, row

    @staticmethod
    def _in_place(value: Value) -> Tuple[Optional[Value], Tuple[int, ...]]:
        """(the stored value or strided view to read in place, or None when ``value`` is an expression that
        must be stored first; its element strides)."""
        if value.stored:
            return value, tuple(value.view.strides)
        if value.view is not None and value.view.base is not None:
            return Value(value.name, value.shape, value.dtype, value.deps, stored=True, view=value.view), tuple(value.view.strides)
        return None, contiguous_strides(value.shape)

    def _operand(self, value: Value, shape: Sequence[int]) -> Tuple[Value, List[int], int]:
        """(stored value, element strides broadcast to ``shape``, element offset): views are read in place,
        expressions are stored once."""
        stored, strides = self._in_place(value)
        if stored is None:
            stored = self.store(value)
        pad = len(shape) - len(value.shape)
        broadcast = [0] * pad + [0 if size == 1 else stride for size, stride in zip(value.shape, strides)]
        return stored, broadcast, stored.view.offset if stored.view.base is not None else 0

    def _matrix_attention(self, out, q, k_past, k_new, v_past, v_new, mask, sinks, scale) -> bool:
        """The long-prefill attention on the matrix cores (``attention_mfma_bf16``); False (nothing
        emitted) when an operand's layout does not allow 16-byte rows."""
        tokens, kv_heads, group, dim = q.shape
        past = k_past.shape[0] if k_past is not None else 0
        keys = past + k_new.shape[0]
        scores_shape = (kv_heads, group, tokens, keys)
        operands = {"q": (q, q.shape), "k_new": (k_new, k_new.shape), "v_new": (v_new, v_new.shape), "mask": (mask, scores_shape),
                    "sinks": (sinks, scores_shape[:3] + (1,))}
        if k_past is not None:
            operands["k_past"], operands["v_past"] = (k_past, k_past.shape), (v_past, v_past.shape)
        # Check every layout before anything is stored: rows of q, K and V contiguous along the head
        # dimension with 16-byte aligned starts, unit key stride in the mask, one sink per head.
        for name, (value, shape) in operands.items():
            stored, strides = self._in_place(value)
            pad = len(shape) - len(value.shape)
            strides = [0] * pad + [0 if size == 1 else stride for size, stride in zip(value.shape, strides)]
            offset = stored.view.offset if stored is not None and stored.view.base is not None else 0
            if name in ("q", "k_new", "v_new", "k_past", "v_past") and (strides[-1] != 1 or any(x % 8 for x in strides[:-1]) or offset % 8):
                return False
            if (name == "mask" and strides[3] != 1) or (name == "sinks" and strides[2] != 0):
                return False
        plan = {name: self._operand(value, shape) for name, (value, shape) in operands.items()}
        plan.setdefault("k_past", None)
        plan.setdefault("v_past", None)
        q_strides, mask_strides, sink_strides = plan["q"][1], plan["mask"][1], plan["sinks"][1]
        k = Kernel(1)
        slot = k.slot(out.name, out.dtype, writable=True, extent=self.extents[out.name])

        def pointer(name: str) -> str:
            entry = plan[name]
            if entry is None:
                entry = plan[name.replace("past", "new")]
            value, _, offset = entry
            root = value.root
            base = k.slot(root.name, root.dtype, extent=self.extents[root.name])
            return f"{base} + {offset}u" if offset else base

        kp = plan["k_past"][1] if plan["k_past"] is not None else plan["k_new"][1]
        vp = plan["v_past"][1] if plan["v_past"] is not None else plan["v_new"][1]
        kn, vn = plan["k_new"][1], plan["v_new"][1]
        k.line("chroma::AttentionOperands a;")
        k.line(f"a.q = {pointer('q')}; a.qt = {q_strides[0]}u; a.qh = {q_strides[1]}u; a.qg = {q_strides[2]}u;")
        k.line(f"a.k_past = {pointer('k_past')}; a.k_new = {pointer('k_new')}; a.v_past = {pointer('v_past')}; a.v_new = {pointer('v_new')};")
        k.line(f"a.kpj = {kp[0]}u; a.kph = {kp[1]}u; a.knj = {kn[0]}u; a.knh = {kn[1]}u;")
        k.line(f"a.vpj = {vp[0]}u; a.vph = {vp[1]}u; a.vnj = {vn[0]}u; a.vnh = {vn[1]}u;")
        k.line(f"a.mask = {pointer('mask')}; a.mt = {mask_strides[2]}u; a.mh = {mask_strides[0]}u; a.mg = {mask_strides[1]}u;")
        k.line(f"a.sinks = {pointer('sinks')}; a.sh = {sink_strides[0]}u; a.sg = {sink_strides[1]}u;")
        k.line(f"a.out = {slot}; a.tokens = {tokens}u; a.past = {past}u; a.keys = {keys}u; a.kv_heads = {kv_heads}u; a.group = {group}u;")
        k.line(f"a.scale = {float_literal(scale)};")
        shared_mask = mask_strides[0] == mask_strides[1] == 0
        if shared_mask and group <= 8:
            # one workgroup per (16-query tile, KV head), one wave per query head: K/V/mask tiles staged once
            live = self._live_blocks(plan["mask"], tokens, keys, tile=(16, 64))
            k.line(f"a.live_blocks = reinterpret_cast<const uint8_t*>({k.slot(live.name, torch.int64, extent=self.extents[live.name])});")
            # a power-of-two scale <= 1 makes the scaled score a bfloat16 value: its rounding is left out
            mantissa, exponent = math.frexp(scale)
            pow2 = mantissa == 0.5 and -64 <= exponent <= 1
            # (head dimensions above 64 would need more registers than three workgroups per CU leave)
            per_wave = ATTENTION_HEADS_PER_WAVE if group % ATTENTION_HEADS_PER_WAVE == 0 and dim <= 64 else 1
            k.min_waves = ATTENTION_HEADS_MIN_BLOCKS if per_wave > 1 else 0
            k.line(f"chroma::attention_heads_mfma_bf16<{dim}, {group}, {'true' if pow2 else 'false'}, {per_wave}>(a);")
            operands = [entry[0] for entry in plan.values() if entry is not None] + [live]
            self.launch(k, (kv_heads, -(-tokens // 16), 1), 64 * group // per_wave, operands, kind="attention_heads")
        else:
            live = self._live_blocks(plan["mask"], tokens, keys) if shared_mask else None
            if live is not None:
                k.line(f"a.live_blocks = reinterpret_cast<const uint8_t*>({k.slot(live.name, torch.int64, extent=self.extents[live.name])});")
            else:
                k.line("a.live_blocks = nullptr;")
            k.line(f"chroma::attention_mfma_bf16<{dim}>(a);")
            # every key block's loads are a round trip and more resident workgroups hide them; five waves per
            # SIMD fit without spills up to D = 64 (D = 128 would spill)
            k.min_waves = 5 if dim <= 64 else 0
            operands = [entry[0] for entry in plan.values() if entry is not None] + ([live] if live is not None else [])
            self.launch(k, (kv_heads * group, -(-tokens // 64), 1), 256, operands, kind="attention_mfma")
        self.fused_attentions += 1
        self.mfma_matmuls += 1
        return True

    def _live_blocks(self, mask_plan, tokens: int, keys: int, tile: Tuple[int, int] = (64, 32)) -> Value:
        """Per (queries x keys) block of a head-independent bfloat16 mask, whether any entry is not -inf:
        computed once per mask and block shape and shared by every attention that reads it. (64, 32)
        blocks also mark the all-+0.0 blocks (``attention_live_blocks``); (16, 64) blocks serve the
        group-shared kernel (``attention_live_tiles``)."""
        value, strides, offset = mask_plan
        key = (value.root.name, offset, strides[2], tokens, keys, tile)
        if key not in self.live_block_tables:
            query_blocks, key_blocks = -(-tokens // tile[0]), -(-keys // tile[1])
            table = self.allocate((-(-query_blocks * key_blocks // 8),), torch.int64)
            k = Kernel(1)
            root = value.root
            base = k.slot(root.name, root.dtype, extent=self.extents[root.name])
            flags = k.slot(table.name, torch.int64, writable=True, extent=self.extents[table.name])
            pointer = f"{base} + {offset}u" if offset else base
            function = "attention_live_blocks" if tile == (64, 32) else "attention_live_tiles"
            assert tile in ((64, 32), (16, 64))
            threads = 256
            if WAVE_LIVE_TILES and tile == (16, 64) and offset % 8 == 0 and strides[2] % 8 == 0:
                function, threads = "attention_live_tiles_wave", 64  # 16-byte loads, one wave per tile
            k.line(f"chroma::{function}({pointer}, {strides[2]}u, {tokens}u, {keys}u, reinterpret_cast<uint8_t*>({flags}));")
            self.launch(k, (query_blocks, key_blocks, 1), threads, [value], kind="attention_blocks")
            self.live_block_tables[key] = table
        return self.live_block_tables[key]

    # ================================================================================= einsum
    def einsum(self, meta, eqn: str, values: Sequence[Value]) -> Value:
        labels, output, sizes, reduction = contraction(eqn, values)
        eqn = eqn.replace(" ", "")
        expert = self._expert_einsum(meta, eqn, labels, sizes, values)
        if expert is not None:
            return expert
        width = math.prod(sizes[letter] for letter in reduction)
        small = len(values) == 2 and meta.dtype in (torch.float32, torch.bfloat16) and width <= SMALL_REDUCTION
        if small:
            # Each output reads ``width`` elements of each operand: an operand whose evaluation costs
            # more than a few loads and operations (such as another small contraction) is stored
            # first, so that chains of small contractions never multiply their re-evaluations.
            operands = [v if width == 1 or self.cost(v) <= SMALL_OPERAND_COST else self.store(v) for v in values]
            return self._small_contraction(meta, labels, output, sizes, reduction, operands)
        matrix = self._matrix_einsum(meta, labels, output, sizes, reduction, values)
        if matrix is not None:
            return matrix
        prepared = []
        for label, value in zip(labels, values):
            reuse = math.prod(sizes[letter] for letter in output if letter not in label)
            # An expression re-evaluated for many outputs is worth one store once the re-evaluations add up.
            if not value.stored and value.view is None and reuse >= 8 and math.prod(value.shape) * reuse >= REUSED_EVALUATIONS:
                value = self.store(value)
            prepared.append(value)
        return self._loop_einsum(meta, labels, output, sizes, reduction, prepared)

    def _small_contraction(self, meta, labels, output, sizes, reduction, values) -> Value:
        """A contraction over at most ``SMALL_REDUCTION`` summed positions (an outer product such as
        position x inverse frequency, or the weighted sum of the selected experts' outputs) as an
        elementwise expression that fuses into its consumers instead of a launch of its own. Each output
        is ``((0 + a0*b0) + a1*b1) + ...`` in the accumulating loop's order (summed labels in sorted order,
        row-major) and rounded once, so it equals the loop kernel's result bit for bit (a negative-zero
        product still comes out as +0)."""
        bf16 = meta.dtype == torch.bfloat16
        reduce_shape = [sizes[letter] for letter in reduction]
        steps = []
        for r in range(math.prod(reduce_shape)):
            digits = []
            for size in reversed(reduce_shape):
                digits.append(r % size)
                r //= size
            steps.append(dict(zip(reduction, [Aff((), d) for d in reversed(digits)])))

        def closure(k: Kernel, coords: List[Aff]) -> tuple:
            node = ("f", 0.0)
            for step in steps:
                by_label = dict(zip(output, coords))
                by_label.update(step)
                factors = [
                    self.read(k, value, [ZERO if size == 1 else by_label[letter] for letter, size in zip(label, value.shape)])
                    for label, value in zip(labels, values)
                ]
                node = ("bin", "add", node, ("bin", "mul", factors[0], factors[1]))
            return ("rnd", node) if bf16 else node

        self.small_contractions += 1
        cost = len(steps) * (2 + sum(self.cost(v) for v in values))
        return self.expr(meta, closure, list(values), cost=cost)

    def _expert_einsum(self, meta, eqn, labels, sizes, values) -> Optional[Value]:
        if not self.blas or eqn not in ("beck,bk->bec", "beck,bek->bec"):
            return None
        source = self.gathers.get(values[0].name)
        if source is None:
            return None
        for label, value in zip(labels, values):
            if any(size != sizes[letter] for letter, size in zip(label, value.shape)):
                return None
        weight, indices = source
        if weight.dtype != meta.dtype or weight.shape[-1] % 4:
            return None
        weight, indices, x = self.contiguous(weight), self.contiguous(indices), values[1]
        if x.dtype != meta.dtype:
            return None
        out = self.allocate(tuple(meta.shape), meta.dtype)
        tokens, selected, channels = out.shape
        inner = weight.shape[-1]
        experts = weight.shape[0]
        per_slot = eqn == "beck,bek->bec"
        per_expert = "true" if per_slot else "false"
        plan = self._stream_plan(1, inner, out.dtype, tokens * selected * channels * inner * ITEMSIZE[out.dtype])
        if (tokens * selected < GROUPED_SLOTS and plan is not None and inner <= STAGED_FLOATS
                and weight.view.offset % (16 // ITEMSIZE[weight.dtype]) == 0):
            # One slot per workgroup row of the grid: the slot's input row (per token or per slot; any
            # view or fused expression, e.g. the gated activation of the first expert product) is
            # evaluated into LDS, then the selected expert's slab is streamed.
            lanes, steps = plan
            blocks_per_slot, threads = self._stream_blocks(channels, lanes, steps), 256
            router = None
            if not per_slot and (blocks_per_slot * tokens * selected <= FOLDED_STAGING_BLOCKS or x.stored or (x.view is not None and x.view.base is not None)):
                router = self._fusible_router(indices, x, tokens, selected, weight.dtype)  # (x is staged as it is: see _stageable)
            if router is not None:
                self._routed_expert_stream(router, out, weight, x, tokens, selected, experts, channels, inner, lanes, steps, blocks_per_slot, threads)
                self.expert_contractions += 1
                return out
            x = self._stageable(x, blocks_per_slot * tokens * selected)
            k = Kernel(1)
            w, idx = self._matrix_slot(k, weight), self._matrix_slot(k, indices)
            out_slot = k.slot(out.name, out.dtype, writable=True, extent=self.extents[out.name])
            k.uses_error = True
            slot = Aff.of(k.atom("blockIdx.y", tokens * selected - 1, prefix="s"))
            if per_slot:
                coords_of = lambda _row: [k.div(slot, selected), k.mod(slot, selected)]
            else:
                coords_of = lambda _row: [k.div(slot, selected)]
            # the slab is requested after the prologue, or before it when the experts are small (see _stream_linear)
            early = channels * inner * ITEMSIZE[weight.dtype] <= EARLY_FETCH_BYTES
            fetch = [f"chroma::StreamStep<{inner}, {lanes}, {steps}, {ctype_of(out.dtype)}> prefetched;",
                     f"chroma::stream_expert_fetch(prefetched, {w}, {idx}, {experts}u, {channels}u, error);"]
            if early:
                for line in fetch:
                    k.line(line)
            self._stage(k, x, 1, inner, coords_of, threads)
            if not early:
                for line in fetch:
                    k.line(line)
            k.line(
                f"chroma::stream_expert_linear<{inner}, {lanes}, {steps}, true, {ctype_of(out.dtype)}, {per_expert}>("
                f"{w}, {idx}, nullptr, xs, {out_slot}, {selected}u, {experts}u, {channels}u, {blocks_per_slot}u, error, prefetched);"
            )
            self.launch(k, (blocks_per_slot, tokens * selected, 1), threads, [weight, indices, x], kind="expert_stream")
            self.expert_contractions += 1
            return out
        if per_slot and not x.stored:
            x = self._activation_epilogue(x) or x
        x = self.contiguous(x)
        if tokens * selected >= GROUPED_SLOTS and inner % (8 if meta.dtype == torch.bfloat16 else 4) == 0 and experts <= 4096:
            self._grouped_experts(out, weight, indices, x, tokens, selected, experts, channels, inner, per_slot)
            self.expert_contractions += 1
            return out
        lanes_per_row = 64
        while lanes_per_row > 1 and inner % (4 * lanes_per_row):
            lanes_per_row //= 2
        k = Kernel(1)
        w, idx, xs = self._matrix_slot(k, weight), self._matrix_slot(k, indices), self._matrix_slot(k, x)
        out_slot = k.slot(out.name, out.dtype, writable=True, extent=self.extents[out.name])
        k.uses_error = True
        rows_per_wave = 64 // lanes_per_row
        blocks_per_slot = -(-(-(-channels // rows_per_wave)) // 4)
        k.line(
            f"chroma::expert_linear<{inner}, {lanes_per_row}, {ctype_of(out.dtype)}, {per_expert}>("
            f"{w}, {idx}, {xs}, {out_slot}, {selected}u, {experts}u, {channels}u, {blocks_per_slot}u, error);"
        )
        self.launch(k, (blocks_per_slot, tokens * selected, 1), 256, [weight, indices, x], kind="expert_linear")
        self.expert_contractions += 1
        return out

    def _fusible_router(self, indices: Value, x: Value, tokens: int, selected: int, dtype) -> Optional[dict]:
        """The router launch that selected ``indices`` when it can be recomputed inside the first expert
        product: it is the last launch, it stages the same row ``x`` the product stages, it routes one row
        per token to ``selected`` experts, and its gate weights are small."""
        router = self.router_launches.get(indices.name)
        if (router is None or router["index"] != len(self.launches) - 1 or router["source"].name != x.name or router["rows"] != tokens
                or router["count"] != selected or router["weight"].dtype != dtype or router["columns"] > 64 or not router["lanes"]
                or router["columns"] * router["inner"] * ITEMSIZE[dtype] > FUSED_ROUTER_BYTES):
            return None
        return router

    def _routed_expert_stream(self, router: dict, out: Value, weight: Value, x: Value, tokens: int, selected: int, experts: int,
                              channels: int, inner: int, lanes: int, steps: int, blocks_per_slot: int, threads: int) -> None:
        """The router and the first expert product in one kernel (``routed_expert_stream``): the router's
        launch is retracted; every workgroup stages its token's row, selects the token's experts itself and
        streams the slab of its slot's expert; one workgroup per token writes the router's outputs."""
        self._retract_last_launch()
        del self.router_launches[router["indices"].name]
        k = Kernel(1)
        ctype = ctype_of(out.dtype)
        slot = Aff.of(k.atom("blockIdx.y", tokens * selected - 1, prefix="s"))
        self._stage(k, x, 1, inner, lambda _row: [k.div(slot, selected)], threads)
        gate = self._matrix_slot(k, router["weight"])
        gate_bias = self._matrix_slot(k, router["bias"]) if router["bias"] is not None else "nullptr"
        outputs = [k.slot(router[name].name, router[name].dtype, writable=True, extent=self.extents[router[name].name])
                   for name in ("logits", "values", "indices", "weights")]
        w = self._matrix_slot(k, weight)
        out_slot = k.slot(out.name, out.dtype, writable=True, extent=self.extents[out.name])
        k.uses_error = True
        k.line(
            f"chroma::routed_expert_stream<{router['columns']}, {router['inner']}, {router['lanes']}, {str(router['largest']).lower()}, "
            f"{inner}, {lanes}, {steps}, {ctype}>(xs, {gate}, {gate_bias}, {outputs[0]}, {outputs[1]}, {outputs[2]}, {outputs[3]}, "
            f"{selected}u, {w}, {out_slot}, {experts}u, {channels}u, {blocks_per_slot}u, error);"
        )
        inputs = [x, router["weight"], weight] + ([router["bias"]] if router["bias"] is not None else [])
        self.launch(k, (blocks_per_slot, tokens * selected, 1), threads, inputs, kind="routed_experts")
        self.routed_experts += 1

    def _matrix_einsum(self, meta, labels, output, sizes, reduction, values) -> Optional[Value]:
        """A batched matrix product on the matrix cores (the reference's ``matrix`` hook, gpu.py:426-435,
        which its CUDA backend leaves to the scalar loop). Taken when the contraction has one row, one
        column and one contracted label, the operands can be read in place with unit stride along the
        contracted label (or along the column label for the right operand), and the product is large
        enough to fill 128 x 128 tiles."""
        found = matrix_axes(labels, output, reduction)
        if not self.blas or found is None:
            return None
        batch, row, column, inner = found
        dtype = meta.dtype
        if any(v.dtype != dtype for v in values) or dtype not in (torch.float32, torch.bfloat16):
            return None
        rows, columns, depth = sizes[row], sizes[column], sizes[inner]
        chunk = 8 if dtype == torch.bfloat16 else 4
        if rows * columns * depth < MATRIX_MIN_WORK or depth % chunk or rows < 16 or columns < 16:
            return None
        out_shape = tuple(meta.shape)
        out_strides = dict(zip(output, contiguous_strides(out_shape)))
        if out_strides[column] != 1:
            return None
        operands, layouts = [], []
        for label, value in zip(labels, values):
            if any(value.shape[label.index(letter)] != sizes[letter] for letter in (row, column, inner) if letter in label):
                return None
            if not value.stored:
                # A strided view (a GQA expand, a head slice) is read in place through its strides.
                value = self.materialize(value) if value.view is not None and value.view.base is not None else self.store(value)
            strides = dict(zip(label, value.view.strides))
            for letter, size in zip(label, value.shape):
                if size == 1:
                    strides[letter] = 0
            operands.append(value)
            layouts.append(strides)
        left, right = layouts
        if left[inner] != 1 or left[row] % chunk:
            return None
        if right[inner] == 1 and right[column] % chunk == 0:
            k_contiguous, ldb = True, right[column]
        elif right[column] == 1 and right[inner] % chunk == 0:
            k_contiguous, ldb = False, right[inner]
        else:
            return None
        for value, strides in zip(operands, layouts):
            if value.view.offset % chunk or any(strides.get(letter, 0) % chunk for letter in batch):
                return None
        out = self.allocate(out_shape, dtype)
        k = Kernel(1)
        batch_sizes = tuple(sizes[letter] for letter in batch) or (1,)
        batches = math.prod(batch_sizes)
        coords = k.unflatten(Aff.of(k.atom("blockIdx.z", batches - 1, prefix="z")), batch_sizes) if batch else []
        pointers, ends = [], []
        spans = ((rows - 1) * left[row] + depth - 1, (columns - 1) * ldb + depth - 1 if k_contiguous else (depth - 1) * ldb + columns - 1)
        for value, strides, span in zip(operands, layouts, spans):
            offset = Aff((), value.view.offset)
            for coord, letter in zip(coords, batch):
                offset = offset + coord.scale(strides.get(letter, 0))
            root = value.root
            slot = k.slot(root.name, root.dtype, extent=self.extents[root.name])
            k.check_bounds(slot, offset + span)
            pointers.append(f"{slot} + ({offset.code()})")
        out_offset = ZERO
        for coord, letter in zip(coords, batch):
            out_offset = out_offset + coord.scale(out_strides[letter])
        out_slot = k.slot(out.name, dtype, writable=True, extent=self.extents[out.name])
        k.check_bounds(out_slot, out_offset + ((rows - 1) * out_strides[row] + columns - 1))
        k.line(
            f"chroma::mfma_gemm<{ctype_of(dtype)}, {str(k_contiguous).lower()}>({pointers[0]}, {left[row]}u, {pointers[1]}, {ldb}u, "
            f"nullptr, {out_slot} + ({out_offset.code()}), {out_strides[row]}u, {rows}u, {columns}u, {depth}u, nullptr, nullptr, "
            f"blockIdx.y * 128u, blockIdx.x * 128u);"
        )
        self.launch(k, (-(-columns // 128), -(-rows // 128), batches), 256, operands, kind="matmul_mfma")
        self.matrix_contractions += 1
        self.mfma_matmuls += 1
        return out

    def _route(self, indices: Value, experts: int) -> Tuple[Value, int]:
        """Group the slots of a router output by expert once; both expert contractions of a layer share it
        (its two tile tables serve 128-slot last tiles and taller ones)."""
        key = (indices.name, experts)
        slots = math.prod(indices.shape)
        tiles = -(-slots // 128) + experts  # chroma::expert_tile_bound
        if key not in self.routes:
            words = 2 * experts + 2 + slots + 2 * tiles + 1 + 2 * tiles
            scratch = self.allocate((-(-words // 2),), torch.int64)
            k = Kernel(1)
            ids = self._matrix_slot(k, indices)
            table = k.slot(scratch.name, torch.int64, writable=True, extent=self.extents[scratch.name])
            k.uses_error = True
            k.line(f"chroma::route_slots({ids}, {slots}u, {experts}u, reinterpret_cast<int32_t*>({table}), error);")
            self.launch(k, 1, 1024, [indices], kind="route", shared=4 * experts)
            self.routes[key] = scratch
        return self.routes[key], tiles

    def _grouped_experts(self, out, weight, indices, x, tokens, selected, experts, channels, inner, per_slot) -> None:
        args = (out, weight, indices, x, tokens, selected, experts, channels, inner, per_slot)
        k, grid, threads, path, scratch = self._grouped_kernel(*args)
        self.launch(k, grid, threads, [weight, x, scratch], kind="experts_mfma")
        self.mfma_matmuls += 1
        self.last_grouped = {"index": len(self.launches) - 1, "args": args, "path": path, "scratch": scratch}

    def _grouped_kernel(self, out, weight, indices, x, tokens, selected, experts, channels, inner, per_slot, activation=None,
                        store_product: bool = True):
        """The grouped expert product's kernel, grid, threads, body path and routing; with ``activation``
        = (value, buffer) the ring body's epilogue writes ``value`` (which reads this product's output)
        into ``buffer``, and the product too unless ``store_product`` is false (``_activation_epilogue``)."""
        path, threads, width, waves, last = 1, 256, 128, 4, 128
        ring = next(((n, w, t) for n, w, t in RING_EXPERT_TILES if channels % n == 0), None)
        if out.dtype == torch.bfloat16 and inner % 32 == 0 and ring is not None:
            path, (width, waves, last) = 3, ring
            threads = 64 * waves
        elif self._direct_gemm(out.dtype, inner):
            path, threads = 2, DIRECT_GEMM_THREADS
        scratch, tiles = self._route(indices, experts)
        k = Kernel(1)
        if path == 3:
            k.min_waves = 1
        elif path == 2:
            k.min_waves = DIRECT_GEMM_BLOCKS
        w, xs = self._matrix_slot(k, weight), self._matrix_slot(k, x)
        table = k.slot(scratch.name, torch.int64, extent=self.extents[scratch.name])
        if activation is None:
            destination, epilogue = k.slot(out.name, out.dtype, writable=True, extent=self.extents[out.name]), ""
        else:
            assert path == 3, "activation epilogues take the ring body"
            self._emit_activation_epilogue(k, out, indices, *activation, tokens, selected, channels, store_product)
            destination, epilogue = f"static_cast<{ctype_of(out.dtype)}*>(nullptr)", ", epilogue"
        k.line(
            f"chroma::grouped_expert_linear<{ctype_of(out.dtype)}, {str(per_slot).lower()}, {path}, {width}, 1, {waves}, {last}>({w}, {xs}, "
            f"{destination}, reinterpret_cast<const int32_t*>({table}), {tokens * selected}u, {selected}u, {experts}u, {channels}u, "
            f"{inner}u{epilogue});"
        )
        return k, 8 * -(-(-(-channels // width) * tiles) // 8), threads, path, scratch

    def _emit_activation_epilogue(self, k: Kernel, product: Value, indices: Value, value: Value, buffer: Value, tokens: int,
                                  selected: int, channels: int, store_product: bool) -> None:
        """The lambda the ring body calls per (slot, 4 consecutive channels c .. c + 3) of ``product``
        [tokens, selected, channels]: it rounds the four sums as the product's store would (and stores
        them when ``store_product``), then evaluates ``value`` [tokens, selected, channels / 2] at channels
        c / 2 and c / 2 + 1 (a gated activation reads channels 2i and 2i + 1 of the product for its channel
        i) and writes both to ``buffer``. The expression is the one a map kernel would evaluate, with every
        read of the product replaced by the lane's rounded sums, and the slot's own expert id (a gather of
        the experts' biases) by the tile's expert, which every slot of the tile is routed to (an id outside
        the experts has already raised the error word in the routing); a read of any other product element
        raises ``_NotFusible``."""
        half = channels // 2
        slot = k.slot(buffer.name, buffer.dtype, writable=True, extent=self.extents[buffer.name])
        with k.block("auto epilogue = [&](uint32_t slot, uint32_t column, const float* sums, uint32_t expert) {", "};"):
            k.line("uint16_t bits[4];")
            k.line("float u[4];")
            k.line("for (int r = 0; r < 4; ++r) {")
            k.line("    bits[r] = chroma::f32_to_bf16(sums[r]);")
            k.line("    u[r] = chroma::bf16_to_f32(bits[r]);  // the product as stored")
            k.line("}")
            b = Aff.of(k.atom(f"slot / {selected}u", tokens - 1, prefix="t"))
            e = Aff.of(k.atom(f"slot % {selected}u", selected - 1, prefix="t"))
            h = k.atom("column / 2u", half - 2, prefix="h")
            row = b.scale(selected * channels) + e.scale(channels)
            if store_product:
                target = k.slot(product.root.name, product.dtype, writable=True, extent=self.extents[product.root.name])
                at = row + Aff.of(h, 2) + product.view.offset
                k.check_bounds(target, at + 3)
                k.line(f"*reinterpret_cast<uint2*>({target} + {at.code()}) = uint2{{uint32_t(bits[0]) | (uint32_t(bits[1]) << 16), "
                       "uint32_t(bits[2]) | (uint32_t(bits[3]) << 16)};")

            def lane_value(address: Aff) -> tuple:
                rest = address.without(h)
                if address.coefficient(h) != 2 or Aff(rest.terms) != row or not 0 <= rest.const < 4:
                    raise _NotFusible(f"the activation reads {product.name}[{address.code()}] outside the lane's four channels")
                return ("lds", "u", Aff((), rest.const))

            slot_id = b.scale(selected) + e + indices.view.offset

            def tile_expert(address: Aff) -> tuple:
                if address != slot_id:
                    raise _NotFusible(f"the activation reads {indices.name}[{address.code()}], not its slot's expert id")
                return ("reg", torch.int64, "int64_t(expert)")

            k.register_reads[product.root.name] = lane_value
            k.register_reads[indices.root.name] = tile_expert
            try:
                names = [k.emit(self.read(k, value, [b, e, Aff.of(h) + p])) for p in (0, 1)]
            finally:
                del k.register_reads[product.root.name]
                del k.register_reads[indices.root.name]
            at = b.scale(selected * half) + e.scale(half) + Aff.of(h)
            k.check_bounds(slot, at + 1)
            k.line(f"*reinterpret_cast<uint32_t*>({slot} + {at.code()}) = uint32_t(chroma::f32_to_bf16({names[0]})) | "
                   f"(uint32_t(chroma::f32_to_bf16({names[1]})) << 16);")

    def _activation_epilogue(self, x: Value) -> Optional[Value]:
        """Store the per-slot operand ``x`` of a second expert product from the epilogue of the first when
        ``x`` is an elementwise expression of that product's output (the gated activation) and the first
        product is the last launch, on the ring body, with ``x`` taking channels 2i and 2i + 1 for its
        channel i (bfloat16). The first product's launch is re-emitted with the epilogue, its output is
        never written (any other read of it fails the compile), and ``x``'s readers read the stored copy.
        Removes the activation's map launch and the round trip of the product through HBM."""
        last = self.last_grouped
        if not ACTIVATION_EPILOGUES or last is None or last["index"] != len(self.launches) - 1 or last["path"] != 3:
            return None
        out, weight, indices, xin, tokens, selected, experts, channels, inner, per_slot = last["args"]
        if (out.name not in self.sources.get(x.name, ()) or x.dtype != torch.bfloat16 or out.dtype != torch.bfloat16
                or tuple(x.shape) != (tokens, selected, channels // 2) or channels % 4):
            return None
        buffer = self.allocate(tuple(x.shape), x.dtype)
        try:
            k, grid, threads, _, scratch = self._grouped_kernel(*last["args"], activation=(x, buffer))
            lean, *_ = self._grouped_kernel(*last["args"], activation=(x, buffer), store_product=False)
        except _NotFusible:
            return None
        self._retract_last_launch()
        self.launch(k, grid, threads, [weight, xin, scratch, x], kind="experts_mfma")
        self.product_stores.append((len(self.launches) - 1, out.root.name, lean, self.launches[-1].grid, threads, (), "experts_mfma"))
        self.epilogue_values[x.name] = buffer
        self.materialized[x.name] = buffer
        self.last_grouped = None
        self.expert_epilogues += 1
        return buffer

    def _drop_unread_product_stores(self) -> None:
        """After lowering: a fused expert launch whose product no later launch binds and no output holds
        takes the variant that does not store the product."""
        for index, product, lean, grid, threads, prologue, kind in self.product_stores:
            if product in self.output_buffers or any(product in launch.buffers for launch in self.launches[index + 1 :]):
                continue
            source = lean.render("KERNEL_NAME", threads, prologue)
            name = self.kernel_names.get(source)
            if name is None:
                name = f"chroma_{kind}_{hashlib.sha256(source.encode()).hexdigest()[:8]}"
                self.kernel_names[source] = name
                self.kernel_sources.append(source.replace("KERNEL_NAME", name, 1))
            old = self.launches[index]
            self.launches[index] = Launch(name, grid, threads, [self.binding_of(buffer) for buffer in lean.slots], old.shared, list(lean.slots))
            if all(launch.kernel != old.kernel for launch in self.launches):
                text = next(src for src, kernel in self.kernel_names.items() if kernel == old.kernel)
                del self.kernel_names[text]
                self.kernel_sources = [text for text in self.kernel_sources if f" {old.kernel}(" not in text]
            self.unstored_products += 1

    def _loop_einsum(self, meta, labels, output, sizes, reduction, values) -> Value:
        out = self.allocate(tuple(meta.shape), meta.dtype)
        out_shape = _shape(out.shape)
        outputs = math.prod(out_shape)
        reduce_shape = tuple(sizes[letter] for letter in reduction) or (1,)
        width = math.prod(reduce_shape) if reduction else 1
        parallel = width >= 512
        k = Kernel(1)
        slot = k.slot(out.name, out.dtype, writable=True, extent=self.extents[out.name])

        def product(out_coords: List[Aff], reduce_coords: List[Aff]) -> str:
            by_label = dict(zip(output, out_coords))
            by_label.update(zip(reduction, reduce_coords))
            factors = []
            for label, value in zip(labels, values):
                coords = [ZERO if size == 1 else by_label[letter] for letter, size in zip(label, value.shape)]
                factors.append(k.emit(self.read(k, value, coords)))
            return f"{factors[0]} * {factors[1]}"

        if parallel:
            groups = 4
            k.line(f"const uint32_t o = blockIdx.x * {groups}u + threadIdx.x / 64u;")
            k.line(f"if (o >= {outputs}u) return;")
            out_coords = k.unflatten(Aff.of(Atom("o", outputs - 1)), out_shape) if meta.shape else []
            k.line("float sum = 0.0f;")
            with k.block(f"for (uint32_t r = threadIdx.x % 64u; r < {width}u; r += 64u) {{"):
                reduce_coords = k.unflatten(Aff.of(Atom("r", width - 1)), reduce_shape)
                k.line(f"sum += {product(out_coords, reduce_coords)};")
            k.line("sum = chroma::wave_sum(sum);")
            k.line("if (threadIdx.x % 64u == 0) {")
            k.indent += 1
            k.store(slot, out.dtype, Aff.of(Atom("o", outputs - 1)), self._lane_values(k, ["sum"]))
            k.indent -= 1
            k.line("}")
            self.launch(k, -(-outputs // groups), 64 * groups, values, kind="contract_waves")
            self.parallel_reductions += 1
        else:
            with k.block(f"for (uint32_t o = blockIdx.x * 256u + threadIdx.x; o < {outputs}u; o += gridDim.x * 256u) {{"):
                out_coords = k.unflatten(Aff.of(Atom("o", outputs - 1)), out_shape) if meta.shape else []
                k.line("float sum = 0.0f;")
                if reduction:
                    with k.block(f"for (uint32_t r = 0; r < {width}u; ++r) {{"):
                        reduce_coords = k.unflatten(Aff.of(Atom("r", width - 1)), reduce_shape)
                        k.line(f"sum += {product(out_coords, reduce_coords)};")
                else:
                    k.line(f"sum += {product(out_coords, [])};")
                k.store(slot, out.dtype, Aff.of(Atom("o", outputs - 1)), self._lane_values(k, ["sum"]))
            self.launch(k, max(1, min(-(-outputs // 256), MAX_GRID)), 256, values, kind="contract")
        return out

    # ================================================================================== finish
    def generate(self, inputs: List[TensorSpec], outputs: List[TensorSpec], stats: Stats) -> GeneratedCode:
        self._drop_unread_product_stores()
        weights_size = len(self.weights)
        workspace_base = _align(weights_size)
        error_base = workspace_base + _align(stats["workspace_bytes"])
        position = error_base + ERROR_REGION
        input_regions, output_regions = [None] * len(inputs), []
        # Small inputs first, then large ones (each in input order): a caller that keeps the large ones on
        # the device (the decoder's caches) uploads all the small ones of a step as one copy.
        for index in sorted(range(len(inputs)), key=lambda i: nbytes(inputs[i]) > SMALL_INPUT_BYTES):
            input_regions[index] = (position, nbytes(inputs[index]))
            position += _align(max(nbytes(inputs[index]), 1))
        for spec in outputs:
            output_regions.append((position, nbytes(spec)))
            position += _align(max(nbytes(spec), 1))
        total = position

        def resolve(binding: Binding) -> int:
            if binding.kind == "weight":
                return binding.offset
            if binding.kind == "input":
                return input_regions[binding.index][0] + binding.offset
            if binding.kind == "output":
                return output_regions[binding.index][0] + binding.offset
            if binding.kind == "arena":
                name = binding.index
                if name in self.output_buffers:
                    return output_regions[self.output_buffers[name]][0] + binding.offset
                return workspace_base + self.allocations[name].offset + binding.offset
            if binding.kind == "error":
                return error_base
            raise AssertionError(binding)

        lines = [
            "chroma-hip-plan 2",  # 2: a 1 KiB error region
            f"arena {total}",
            f"weights {weights_size}",
            f"error {error_base}",
        ]
        lines += [f"input {i} {offset} {size}" for i, (offset, size) in enumerate(input_regions)]
        lines += [f"output {i} {offset} {size}" for i, (offset, size) in enumerate(output_regions)]
        for launch in self.launches:
            offsets = [resolve(b) for b in launch.bindings] + [error_base]
            grid = " ".join(map(str, launch.grid))
            lines.append(f"launch {launch.kernel} {grid} {launch.block} {launch.shared} {len(offsets)} {' '.join(map(str, offsets))}")
        stats = dict(
            stats,
            backend="hip",
            input_bytes=sum(map(nbytes, inputs)),
            hip_buffer_bytes=total,
            parallel_reductions=self.parallel_reductions,
            expert_contractions=self.expert_contractions,
            tiled_matmuls=self.tiled_matmuls,
            skinny_matmuls=self.skinny_matmuls,
            mfma_matmuls=self.mfma_matmuls,
            fused_attentions=self.fused_attentions,
            fused_routers=self.fused_routers,
            routed_experts=self.routed_experts,
            expert_epilogues=self.expert_epilogues,
            unstored_products=self.unstored_products,
            reused_maps=self.reused_maps,
            norm_epilogues=self.norm_epilogues,
            weight_prefetches=self.weight_prefetches,
            small_contractions=self.small_contractions,
            attention_epilogues=self.attention_epilogues,
            write_through_stores=len(self.write_through_stores),
            unique_kernels=len(self.kernel_sources),
            launches=len(self.launches),
        )
        source = "#include <chroma_hip/kernels.h>\n\n" + "\n\n".join(self.kernel_sources) + "\n"
        plan = "\n".join(lines) + "\n"
        return GeneratedCode({"model.hip": source, "model.plan": plan}, "model.hip", [], stats, inputs, outputs, self.weights)
