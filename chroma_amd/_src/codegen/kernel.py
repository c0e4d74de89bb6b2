"""A small compiler from fused value expressions to straight-line HIP code.

Every generated kernel computes ``Lanes`` neighbouring elements per thread along the innermost axis
(SIMD within a thread). Values are built as hash-consed expression nodes over *affine* integer
addresses, so that each generated statement is emitted once per kernel and the index arithmetic is
simplified symbolically:

* an ``Atom`` is a named integer with a known inclusive maximum; it is *uniform* (one value per thread)
  or *varying* (one value per lane); the vector atom's lane ``l`` is ``base + l``;
* an ``Aff`` is ``const + sum(coef * atom)`` with non-negative coefficients;
* ``div``/``mod`` by a constant fold exactly when the affine form's bounds allow it (e.g. a transpose,
  a reshape that splits or merges axes, or a slice) and only otherwise declare an opaque atom;
* a load whose address is ``vector atom + aligned uniform part`` becomes one 128-bit (or 64-bit) load,
  a load with no varying part is issued once for all lanes, anything else is issued per lane.

Floating-point nodes compute in float32 (bfloat16 values widen exactly and are rounded back with the
host's round-to-nearest-even rule wherever a bfloat16 result is produced); int64 nodes only move data.
"""

from __future__ import annotations

import contextlib
import itertools
import math
from typing import Dict, Iterator, List, Optional, Sequence, Set, Tuple, Union

import torch

from chroma_amd._src.value import contiguous_strides

U32_LIMIT = 2**32 - 1


class Atom:
    __slots__ = ("name", "hi", "varying", "vector")

    def __init__(self, name: str, hi: int, varying: bool = False, vector: bool = False) -> None:
        self.name, self.hi, self.varying, self.vector = name, int(hi), varying, vector

    def code(self, lane: int) -> str:
        if self.vector:
            return self.name if lane == 0 else f"({self.name} + {lane}u)"
        if self.varying:
            return f"{self.name}_{lane}"
        return self.name

    def __repr__(self) -> str:
        return self.name


class Aff:
    """``const + sum(coef * atom)`` with integer coefficients > 0 (immutable, hashable by value)."""

    __slots__ = ("terms", "const", "_key")

    def __init__(self, terms: Sequence[Tuple[Atom, int]] = (), const: int = 0) -> None:
        merged: Dict[str, List] = {}
        for atom, coef in terms:
            if coef == 0 or atom.hi == 0:
                continue
            if atom.name in merged:
                merged[atom.name][1] += coef
            else:
                merged[atom.name] = [atom, coef]
        self.terms = tuple(sorted(((a, c) for a, c in merged.values() if c), key=lambda t: t[0].name))
        self.const = int(const)
        self._key = (tuple((a.name, c) for a, c in self.terms), self.const)

    @staticmethod
    def of(atom: Atom, coef: int = 1) -> "Aff":
        return Aff(((atom, coef),))

    def __add__(self, other: Union["Aff", int]) -> "Aff":
        if isinstance(other, int):
            return Aff(self.terms, self.const + other)
        return Aff(self.terms + other.terms, self.const + other.const)

    def scale(self, factor: int) -> "Aff":
        return Aff(tuple((a, c * factor) for a, c in self.terms), self.const * factor)

    def hi(self) -> int:
        return self.const + sum(c * a.hi for a, c in self.terms)

    @property
    def varying(self) -> bool:
        return any(a.varying for a, _ in self.terms)

    def coefficient(self, atom: Atom) -> int:
        for a, c in self.terms:
            if a is atom or a.name == atom.name:
                return c
        return 0

    def without(self, atom: Atom) -> "Aff":
        return Aff(tuple((a, c) for a, c in self.terms if a.name != atom.name), self.const)

    def code(self, lane: int = 0, wide: Optional[bool] = None) -> str:
        wide = self.hi() > U32_LIMIT if wide is None else wide
        cast = "(uint64_t)" if wide else ""
        parts = []
        for atom, coef in self.terms:
            term = f"{cast}{atom.code(lane)}"
            parts.append(term if coef == 1 else f"{term} * {coef}u")
        if self.const or not parts:
            parts.append(f"{self.const}u" if not wide else f"{self.const}ull")
        return " + ".join(parts)

    def __hash__(self) -> int:
        return hash(self._key)

    def __eq__(self, other: object) -> bool:
        return isinstance(other, Aff) and self._key == other._key

    def __repr__(self) -> str:
        return self.code()


ZERO = Aff()


def ctype_of(dtype: torch.dtype) -> str:
    return {torch.float32: "float", torch.bfloat16: "uint16_t", torch.int64: "int64_t"}[dtype]


def is_int(dtype: torch.dtype) -> bool:
    return dtype == torch.int64


# Expression nodes are tuples (hash-consed through the kernel's memo):
#   ("ld", slot, dtype, aff)   ("f", value)   ("i", value)   ("un", op, x)   ("bin", op, x, y)
#   ("rnd", x)   ("sel", cond, x, y)   ("cmp", op, aff_a, aff_b, constant)   ("cases", tests, parts)
#   ("reg", dtype, code): a value the surrounding code already holds (C expression ``code``)
Node = tuple

UNARY_CODE = {
    "neg": "(-{x})",
    "abs": "__builtin_fabsf({x})",
    "exp": "chroma::fast_exp({x})",
    "sin": "sinf({x})",
    "cos": "cosf({x})",
    "sqrt": "sqrtf({x})",
    "rsqrt": "(1.0f / sqrtf({x}))",
    "reciprocal": "(1.0f / {x})",
    "sigmoid": "chroma::fast_sigmoid({x})",
    "tanh": "chroma::fast_tanh({x})",
    "silu": "chroma::fast_silu({x})",
    "square": "({x} * {x})",
    "log": "logf({x})",
}
BINARY_CODE = {
    "add": "({a} + {b})",
    "sub": "({a} - {b})",
    "mul": "({a} * {b})",
    "div": "({a} / {b})",
    "pow": "powf({a}, {b})",
    "lowclamp": "({a} < {b} ? {b} : {a})",  # NaN-preserving clamp from below
    "highclamp": "({a} > {b} ? {b} : {a})",  # NaN-preserving clamp from above
    "max": "__builtin_fmaxf({a}, {b})",
}


def float_literal(value: float) -> str:
    value = float(value)
    if math.isnan(value):
        return "__builtin_nanf(\"\")"
    if math.isinf(value):
        return "(-__builtin_inff())" if value < 0 else "__builtin_inff()"
    return repr(value) + "f"


class Kernel:
    """Collects the parameters and body of one generated kernel."""

    def __init__(self, lanes: int = 1) -> None:
        self.lanes = lanes
        self.lines: List[str] = []
        self.slots: Dict[str, Tuple[str, torch.dtype, bool]] = {}  # buffer -> (param name, dtype, writable)
        self.extents: Dict[str, int] = {}  # param name -> element count of the buffer behind it
        self.ids = itertools.count()
        self.atoms: Dict[tuple, Atom] = {}
        self.nodes: Dict[Node, Union[str, List[str]]] = {}
        self.values: Dict[tuple, Node] = {}  # (value name, coordinate keys) -> node
        self.indent = 1
        self.definitions: Dict[str, Tuple[str, "Aff", int]] = {}  # opaque atom -> (op, operand, constant)
        self.uses_error = False
        # Workgroups per compute unit the register allocation must leave room for (__launch_bounds__'s
        # second argument; 0: the compiler's choice): with 256 threads, n workgroups are n waves per SIMD. A
        # latency-bound kernel trades a few registers for more resident workgroups.
        self.min_waves = 0
        self.streaming = False  # vector float stores bypass the caches (results read by later kernels only)
        # Vector loads from buffers of at least this many bytes bypass the caches too (0: never). Set on
        # kernels that read each element of their large operands once.
        self.streaming_loads = 0
        # Load hoisting for unrolled chunk loops: while ``load_log`` is a list, every vector load is also
        # kept in ``array[load_index]`` and logged as (array, C type); while ``load_replay`` is set, the
        # same vector loads (met in the same order) read those arrays instead of memory.
        self.load_log: Optional[List[Tuple[str, str]]] = None
        self.load_replay: Optional[Iterator[str]] = None
        self.load_index = "c"
        self.shared: List[str] = []
        # Arena buffers this kernel computes from their expressions instead of loading (buffer -> Value),
        # and the subset whose stores this kernel performs.
        self.scalar_lane_loads = 0  # varying loads that could not be one vector access
        self.unstored: Dict[str, object] = {}
        self.resolved_stores: List[str] = []
        # Values whose elements this kernel has evaluated into a __shared__ float array (value -> array),
        # in row-major order; reads of them become LDS reads ("lds" nodes).
        self.staged_values: Dict[str, str] = {}
        # Stored buffers whose reads resolve to nodes the kernel already holds (buffer -> address -> node),
        # e.g. an epilogue reading the product it is storing.
        self.register_reads: Dict[str, object] = {}

    # -- parameters ------------------------------------------------------------------------------
    def slot(self, buffer: str, dtype: torch.dtype, writable: bool = False, extent: Optional[int] = None) -> str:
        if buffer in self.slots:
            name, existing, was_writable = self.slots[buffer]
            if writable and not was_writable:
                self.slots[buffer] = (name, existing, True)
            return name
        name = f"b{len(self.slots)}"
        self.slots[buffer] = (name, dtype, writable)
        if extent is not None:
            self.extents[name] = extent
        return name

    def check_bounds(self, slot: str, aff: Aff) -> None:
        """Every generated address is proven in bounds at compile time from the atoms' ranges."""
        extent = self.extents.get(slot)
        if extent is not None and aff.hi() >= extent:
            raise AssertionError(f"generated access {slot}[{aff.code()}] may exceed {extent} elements (bound {aff.hi()})")

    def parameters(self) -> List[str]:
        params = []
        for name, dtype, writable in self.slots.values():
            const = "" if writable else "const "
            params.append(f"{const}{ctype_of(dtype)}* __restrict__ {name}")
        params.append("unsigned int* __restrict__ error")
        return params

    # -- statements ------------------------------------------------------------------------------
    def line(self, text: str) -> None:
        self.lines.append("    " * self.indent + text)

    @contextlib.contextmanager
    def block(self, opener: str, closer: str = "}") -> Iterator[None]:
        """A nested C block; atoms and nodes declared inside are forgotten when it closes."""
        self.line(opener)
        saved = (dict(self.atoms), dict(self.nodes), dict(self.values))
        self.indent += 1
        try:
            yield
        finally:
            self.indent -= 1
            self.atoms, self.nodes, self.values = saved
            self.line(closer)

    def fresh(self, prefix: str) -> str:
        return f"{prefix}{next(self.ids)}"

    # -- atoms -----------------------------------------------------------------------------------
    def atom(self, code: str, hi: int, *, prefix: str = "a") -> Atom:
        """Declare a uniform integer from C code."""
        key = ("code", code)
        if key in self.atoms:
            return self.atoms[key]
        atom = Atom(self.fresh(prefix), hi)
        ctype = "uint64_t" if hi > U32_LIMIT else "uint32_t"
        self.line(f"const {ctype} {atom.name} = {code};")
        self.atoms[key] = atom
        return atom

    def vector_atom(self, base_code: str, hi: int) -> Atom:
        """Declare the lane atom: lane l has value base + l; ``base`` is a multiple of ``lanes``."""
        atom = Atom(self.fresh("j"), hi, varying=self.lanes > 1, vector=True)
        ctype = "uint64_t" if hi > U32_LIMIT else "uint32_t"
        self.line(f"const {ctype} {atom.name} = {base_code};")
        return atom

    def loop_atom(self, name: str, hi: int) -> Atom:
        return Atom(name, hi)

    def _opaque(self, key: tuple, aff: Aff, fmt: str, hi: int) -> Aff:
        if key in self.atoms:
            return Aff.of(self.atoms[key])
        wide = aff.hi() > U32_LIMIT
        ctype = "uint64_t" if max(hi, aff.hi()) > U32_LIMIT else "uint32_t"
        op = key[0]
        if aff.varying:
            atom = Atom(self.fresh("a"), hi, varying=True)
            for lane in range(self.lanes):
                self.line(f"const {ctype} {atom.name}_{lane} = {fmt.format(aff.code(lane, wide))};")
        else:
            atom = Atom(self.fresh("a"), hi)
            self.line(f"const {ctype} {atom.name} = {fmt.format(aff.code(0, wide))};")
        self.definitions[atom.name] = (op, aff, key[2])
        self.atoms[key] = atom
        return Aff.of(atom)

    def derived(self, aff: Aff, fmt: str, hi: int) -> Aff:
        """An integer computed from ``aff`` by the C template ``fmt`` (``{}`` = the affine value), with
        inclusive maximum ``hi``; one value per lane when ``aff`` varies across lanes."""
        return self._opaque(("derived", aff, fmt), aff, fmt, hi)

    def div(self, aff: Aff, divisor: int) -> Aff:
        if divisor == 1:
            return aff
        if aff.hi() < divisor:
            return ZERO
        quotient, remainder = [], []
        for atom, coef in aff.terms:
            q, r = divmod(coef, divisor)
            if q:
                quotient.append((atom, q))
            if r:
                remainder.append((atom, r))
        low = Aff(remainder, aff.const % divisor)
        if low.hi() < divisor:
            return Aff(quotient, aff.const // divisor)
        split = self._split_terms(low, divisor)
        if split is not None:
            return Aff(quotient + split[0], aff.const // divisor)
        return self._opaque(("div", aff, divisor), aff, f"({{}}) / {divisor}u", aff.hi() // divisor)

    def _split_terms(self, low: Aff, divisor: int) -> Optional[Tuple[List[Tuple[Atom, int]], Aff]]:
        """``low`` (every coefficient below ``divisor``) as divisor * q + r with 0 <= r < divisor, by
        writing each uniform term c * a whose coefficient divides the divisor as
        divisor * (a / m) + c * (a % m), m = divisor / c: returns (q's terms, r), or None when the rest
        still reaches the divisor. (a / m and a % m are uniform: computed once, shifts for powers of two.)
        Folds the head-major addresses views produce, e.g. (64 * head + j) / 512 = head / 8 for j < 64."""
        quotient: List[Tuple[Atom, int]] = []
        rest = Aff((), low.const)
        changed = False
        for atom, coef in low.terms:
            if coef > 1 and divisor % coef == 0 and not atom.varying and atom.hi >= divisor // coef:
                m = divisor // coef
                whole = Aff.of(atom)
                quotient += self._opaque(("div", whole, m), whole, f"({{}}) / {m}u", atom.hi // m).terms
                rest = rest + self._opaque(("mod", whole, m), whole, f"({{}}) % {m}u", m - 1).scale(coef)
                changed = True
            else:
                rest = rest + Aff(((atom, coef),))
        if not changed or rest.hi() >= divisor:
            return None
        return quotient, rest

    def mod(self, aff: Aff, modulus: int) -> Aff:
        if modulus == 1:
            return ZERO
        if aff.hi() < modulus:
            return aff
        reduced = Aff([(a, c % modulus) for a, c in aff.terms], aff.const % modulus)
        if reduced.hi() < modulus:
            return reduced
        split = self._split_terms(reduced, modulus)
        if split is not None:
            return split[1]
        # aff and its reduced form differ by a multiple of the modulus: the remainder of the reduced form
        # (fewer terms, and shared with any other address that reduces to it)
        return self._opaque(("mod", reduced, modulus), reduced, f"({{}}) % {modulus}u", min(modulus - 1, reduced.hi()))

    def unflatten(self, flat: Aff, shape: Sequence[int]) -> List[Aff]:
        coords = []
        for size, stride in zip(shape, contiguous_strides(shape)):
            coords.append(ZERO if size == 1 else self.mod(self.div(flat, stride), size))
        return coords

    @staticmethod
    def flatten(coords: Sequence[Aff], shape: Sequence[int]) -> Aff:
        total = ZERO
        for coord, size, stride in zip(coords, shape, contiguous_strides(shape)):
            if size != 1:
                total = total + coord.scale(stride)
        return total

    def index_atom(self, value: Node, count: int, negative: bool) -> Aff:
        """A gathered row index: checked against ``count`` (raising the error word) before use."""
        key = ("index", value, count, negative)
        if key in self.atoms:
            return Aff.of(self.atoms[key])
        self.uses_error = True
        names = self.emit(value)
        ctype = "uint64_t" if count - 1 > U32_LIMIT else "uint32_t"
        call = "({ctype})chroma::checked_index({v}, {count}ull, {neg}, error)"
        neg = "true" if negative else "false"
        if isinstance(names, list):
            atom = Atom(self.fresh("g"), count - 1, varying=True)
            for lane, name in enumerate(names):
                self.line(f"const {ctype} {atom.name}_{lane} = " + call.format(ctype=ctype, v=name, count=count, neg=neg) + ";")
        else:
            atom = Atom(self.fresh("g"), count - 1)
            self.line(f"const {ctype} {atom.name} = " + call.format(ctype=ctype, v=names, count=count, neg=neg) + ";")
        self.atoms[key] = atom
        return Aff.of(atom)

    # -- nodes -----------------------------------------------------------------------------------
    @staticmethod
    def node_is_int(node: Node) -> bool:
        tag = node[0]
        if tag == "ld":
            return is_int(node[2])
        if tag == "i":
            return True
        if tag == "reg":
            return is_int(node[1])
        if tag == "sel":
            return Kernel.node_is_int(node[2])
        if tag == "cases":
            return Kernel.node_is_int(node[2][0])
        return False

    def _vector_aligned(self, aff: Aff, vector: Atom, lanes: int = 0) -> bool:
        lanes = lanes or self.lanes
        rest = aff.without(vector)
        if rest.varying or aff.coefficient(vector) != 1:
            return False
        return all(c % lanes == 0 for _, c in rest.terms) and rest.const % lanes == 0

    def emit(self, node: Node) -> Union[str, List[str]]:
        """Emit ``node`` (and its operands); returns one C name (uniform) or one per lane (varying)."""
        if node in self.nodes:
            return self.nodes[node]
        tag = node[0]
        if tag == "f":
            result: Union[str, List[str]] = float_literal(node[1])
        elif tag == "i":
            result = f"int64_t({int(node[1])}ll)"
        elif tag == "reg":
            result = node[2]
        elif tag == "ld":
            result = self._emit_load(node)
        elif tag == "lds":
            _, array, aff = node
            if aff.varying:
                result = []
                for lane in range(self.lanes):
                    result.append(self.fresh("s"))
                    self.line(f"const float {result[-1]} = {array}[{aff.code(lane)}];")
            else:
                result = self.fresh("s")
                self.line(f"const float {result} = {array}[{aff.code()}];")
        elif tag == "cmp":
            result = self._emit_compare(node)
        elif tag == "cases":
            result = self._emit_cases(node)
        else:
            operands = [self.emit(part) for part in node[2:]] if tag in ("un", "bin") else [self.emit(part) for part in node[1:]]
            varying = any(isinstance(o, list) for o in operands)
            if tag == "rnd" and varying and self.lanes % 2 == 0:
                # bfloat16 rounding of an intermediate, two lanes per v_cvt_pk_bf16_f32 (a NaN keeps being a
                # NaN; stores canonicalise it through f32_to_bf16)
                names = []
                for lane in range(0, self.lanes, 2):
                    first, second = self.fresh("n"), self.fresh("n")
                    self.line(f"float {first} = {operands[0][lane]}, {second} = {operands[0][lane + 1]};")
                    self.line(f"chroma::round_bf16_pair({first}, {second});")
                    names += [first, second]
                self.nodes[node] = names
                return names
            lanes = range(self.lanes) if varying else [None]
            names = []
            for lane in lanes:
                args = [o[lane] if isinstance(o, list) else o for o in operands]
                if tag == "un":
                    code = UNARY_CODE[node[1]].format(x=args[0])
                elif tag == "bin":
                    code = BINARY_CODE[node[1]].format(a=args[0], b=args[1])
                elif tag == "rnd":
                    code = f"chroma::round_bf16_fast({args[0]})"
                elif tag == "sel":
                    code = f"({args[0]} ? {args[1]} : {args[2]})"
                else:
                    raise AssertionError(node)
                ctype = "int64_t" if self.node_is_int(node) else ("bool" if tag == "cmp" else "float")
                name = self.fresh("n")
                self.line(f"const {ctype} {name} = {code};")
                names.append(name)
            result = names if varying else names[0]
        self.nodes[node] = result
        return result

    def hoist_loads(self, node: Node) -> None:
        """Emit every memory load of ``node`` before any of its arithmetic (the loads of a piecewise part
        are hoisted to the top of that part's branch instead), so they are all requested at once: emitted
        where the expression needs them, a load after a libm call (whose branches split basic blocks) waits
        a round trip of its own. Every generated address is proven in bounds for its atoms' whole ranges
        and gathered indices are checked when the expression is built, so an earlier load reads nothing
        the expression would not have read. Not while chunk loads are logged or replayed (their order is
        fixed)."""
        if self.load_log is not None or self.load_replay is not None:
            return
        stack, seen = [node], set()
        while stack:
            current = stack.pop()
            if not isinstance(current, tuple) or current in seen:
                continue
            seen.add(current)
            tag = current[0]
            if tag == "ld":
                self.emit(current)
            elif tag in ("un", "bin"):
                stack.extend(reversed(current[2:]))
            elif tag in ("rnd", "sel"):
                stack.extend(reversed(current[1:]))

    @staticmethod
    def load_nodes(node: Node) -> List[Node]:
        """The memory loads of ``node`` outside its piecewise parts, each once, in a fixed order (the same
        for two expressions of the same structure)."""
        order: List[Node] = []
        seen: Set[Node] = set()

        def walk(current) -> None:
            if not isinstance(current, tuple) or current in seen:
                return
            seen.add(current)
            tag = current[0]
            if tag == "ld":
                order.append(current)
            elif tag in ("un", "bin"):
                for part in current[2:]:
                    walk(part)
            elif tag in ("rnd", "sel"):
                for part in current[1:]:
                    walk(part)

        walk(node)
        return order

    def _emit_cases(self, node: Node) -> Union[str, List[str]]:
        """("cases", tests, parts): parts[i] for the first true tests[i] (the last part otherwise). With
        uniform tests only the selected part is evaluated (one branch each); tests that vary across lanes
        fall back to selects over every part."""
        _, tests, parts = node
        if any(test[2].varying or test[3].varying for test in tests):
            chained = parts[-1]
            for test, part in zip(reversed(tests), reversed(parts[:-1])):
                chained = ("sel", test, part, chained)
            return self.emit(chained)
        ctype = "int64_t" if self.node_is_int(parts[0]) else "float"
        base = self.fresh("c")
        # One result per lane (parts may vary across lanes even when the tests do not).
        names = [base] if self.lanes == 1 else [f"{base}_{lane}" for lane in range(self.lanes)]
        self.line(f"{ctype} {', '.join(names)};")
        conditions = [self.emit(test) for test in tests]
        for i, part in enumerate(parts):
            if i < len(tests):
                self.line(("if (" if i == 0 else "} else if (") + f"{conditions[i]}) {{")
            else:
                self.line("} else {" if tests else "{")
            saved = (dict(self.atoms), dict(self.nodes), dict(self.values))
            self.indent += 1
            self.hoist_loads(part)
            value = self.emit(part)
            for lane, name in enumerate(names):
                self.line(f"{name} = {value[lane] if isinstance(value, list) else value};")
            self.indent -= 1
            self.atoms, self.nodes, self.values = saved
        self.line("}")
        return names if self.lanes > 1 else base

    def _emit_compare(self, node: Node) -> Union[str, List[str]]:
        _, op, left, right, constant = node
        varying = left.varying or right.varying
        names = []
        for lane in range(self.lanes) if varying else [0]:
            name = self.fresh("p")
            self.line(f"const bool {name} = int64_t({left.code(lane, True)}) - int64_t({right.code(lane, True)}) {op} {constant}ll;")
            names.append(name)
        return names if varying else names[0]

    def _emit_load(self, node: Node) -> Union[str, List[str]]:
        _, slot, dtype, aff = node
        self.check_bounds(slot, aff)
        if any(buffer in self.slots and self.slots[buffer][0] == slot for buffer in self.unstored):
            # the first workgroup is writing this buffer during the kernel: a load would race with it
            raise AssertionError(f"generated load from {slot}, which this kernel computes in place")
        vector = next((a for a, _ in aff.terms if a.vector), None)
        wide = aff.hi() > U32_LIMIT

        def widen(code: str) -> str:
            return f"chroma::bf16_to_f32({code})" if dtype == torch.bfloat16 else code

        ctype = "int64_t" if is_int(dtype) else "float"
        if not aff.varying:
            name = self.fresh("l")
            self.line(f"const {ctype} {name} = {widen(f'{slot}[{aff.code(0, wide)}]')};")
            return name
        names = [self.fresh("l") for _ in range(self.lanes)]
        if (vector is not None and self.lanes == 8 and not is_int(dtype) and not self._vector_aligned(aff, vector)
                and self._vector_aligned(aff, vector, 4)):
            # 8 lanes on a 4-element alignment: two 4-lane loads
            base = aff.code(0, wide)
            for half in range(2):
                at = f"({base}) + 4u" if half else base
                raw = self.fresh("v")
                if dtype == torch.float32:
                    self.line(f"const float4 {raw} = *reinterpret_cast<const float4*>({slot} + {at});")
                    for lane in range(4):
                        self.line(f"const float {names[4 * half + lane]} = {raw}.{'xyzw'[lane]};")
                else:
                    self.line(f"const uint2 {raw} = *reinterpret_cast<const uint2*>({slot} + {at});")
                    for lane in range(4):
                        word = f"{raw}.{'xy'[lane // 2]}"
                        bits = f"(uint16_t)({word} & 0xffffu)" if lane % 2 == 0 else f"(uint16_t)({word} >> 16)"
                        self.line(f"const float {names[4 * half + lane]} = chroma::bf16_to_f32({bits});")
            return names
        if vector is not None and self.lanes > 1 and not is_int(dtype) and self._vector_aligned(aff, vector):
            base = aff.code(0, wide)
            raw = self.fresh("v")
            itemsize = 4 if dtype == torch.float32 else 2
            streaming = 0 < self.streaming_loads <= self.extents.get(slot, 0) * itemsize
            if dtype == torch.float32 and self.lanes == 8:
                # two 16-byte loads
                halves = [self.fresh("v"), self.fresh("v")]
                for half, name in enumerate(halves):
                    at = f"{base} + {4 * half}u" if half else base
                    load = f"chroma::load_streaming4({slot} + {at})" if streaming else f"*reinterpret_cast<const float4*>({slot} + {at})"
                    self.line(f"const {'chroma::float4_nt' if streaming else 'float4'} {name} = {load};")
                for lane, name in enumerate(names):
                    self.line(f"const float {name} = {halves[lane // 4]}.{'xyzw'[lane % 4]};")
                return names
            if dtype == torch.float32:
                vtype = {2: "float2", 4: "float4"}[self.lanes]
                if streaming:
                    vtype = f"chroma::{vtype}_nt"
                    load = f"chroma::load_streaming{self.lanes}({slot} + {base})"
                else:
                    load = f"*reinterpret_cast<const {vtype}*>({slot} + {base})"
            else:
                vtype = {2: "uint32_t", 4: "uint2", 8: "uint4"}[self.lanes]
                if streaming:
                    vtype = {2: "uint32_t", 4: "chroma::uint2_nt", 8: "chroma::uint4_nt"}[self.lanes]
                    load = f"chroma::load_streaming_bf16x{self.lanes}({slot} + {base})"
                else:
                    load = f"*reinterpret_cast<const {vtype}*>({slot} + {base})"
            if self.load_replay is not None:
                self.line(f"const {vtype} {raw} = {next(self.load_replay)}[{self.load_index}];")
            else:
                self.line(f"const {vtype} {raw} = {load};")
                if self.load_log is not None:
                    array = self.fresh("pre")
                    self.load_log.append((array, vtype))
                    self.line(f"{array}[{self.load_index}] = {raw};")
            if dtype == torch.float32:
                fields = "xyzw"
                for lane, name in enumerate(names):
                    self.line(f"const float {name} = {raw}.{fields[lane]};")
            else:
                words = [f"{raw}"] if self.lanes == 2 else [f"{raw}.{f}" for f in "xyzw"[: self.lanes // 2]]
                for lane, name in enumerate(names):
                    word = words[lane // 2]
                    bits = f"(uint16_t)({word} & 0xffffu)" if lane % 2 == 0 else f"(uint16_t)({word} >> 16)"
                    self.line(f"const float {name} = chroma::bf16_to_f32({bits});")
            return names
        self.scalar_lane_loads += 1
        for lane, name in enumerate(names):
            self.line(f"const {ctype} {name} = {widen(f'{slot}[{aff.code(lane, wide)}]')};")
        return names

    def store(self, slot: str, dtype: torch.dtype, aff: Aff, node: Node) -> None:
        """Write ``node`` (one value per lane) to ``slot[aff]``; contiguous aligned lanes use one store."""
        self.check_bounds(slot, aff)
        values = self.emit(node)
        per_lane = values if isinstance(values, list) else [values] * self.lanes
        vector = next((a for a, _ in aff.terms if a.vector), None)
        wide = aff.hi() > U32_LIMIT

        def narrow(code: str) -> str:
            return f"chroma::f32_to_bf16({code})" if dtype == torch.bfloat16 else code

        if vector is not None and self.lanes > 1 and not is_int(dtype) and self._vector_aligned(aff, vector):
            base = aff.code(0, wide)
            if dtype == torch.float32 and self.lanes == 8:
                for half in range(2):
                    at = f"{base} + {4 * half}u" if half else base
                    quad = per_lane[4 * half : 4 * half + 4]
                    if self.streaming:
                        self.line(f"chroma::store_streaming4({slot} + {at}, {', '.join(quad)});")
                    else:
                        self.line(f"*reinterpret_cast<float4*>({slot} + {at}) = float4{{{', '.join(quad)}}};")
                return
            if dtype == torch.float32:
                if self.streaming:
                    self.line(f"chroma::store_streaming{self.lanes}({slot} + {base}, {', '.join(per_lane)});")
                    return
                vtype = {2: "float2", 4: "float4"}[self.lanes]
                self.line(f"*reinterpret_cast<{vtype}*>({slot} + {base}) = {vtype}{{{', '.join(per_lane)}}};")
            else:
                bits = [f"uint32_t({narrow(v)})" for v in per_lane]
                words = [f"({bits[i]} | ({bits[i + 1]} << 16))" for i in range(0, self.lanes, 2)]
                vtype = {2: "uint32_t", 4: "uint2", 8: "uint4"}[self.lanes]
                value = words[0] if self.lanes == 2 else f"{vtype}{{{', '.join(words)}}}"
                self.line(f"*reinterpret_cast<{vtype}*>({slot} + {base}) = {value};")
            return
        lanes = range(self.lanes) if aff.varying else [0]
        for lane in lanes:
            self.line(f"{slot}[{aff.code(lane, wide)}] = {narrow(per_lane[lane])};")

    def render(self, name: str, launch_bounds: int, prologue: Sequence[str] = ()) -> str:
        bounds = f"{launch_bounds}, {self.min_waves}" if self.min_waves else f"{launch_bounds}"
        head = f'extern "C" __global__ void __launch_bounds__({bounds}) {name}({", ".join(self.parameters())}) {{'
        body = [f"    {line}" for line in prologue] + self.lines
        return "\n".join([head, *body, "}"])


def choose_lanes(extent: int, dtype: torch.dtype, limit: int = 4) -> int:
    """Lanes per thread along an innermost extent: the widest of ``limit`` (at most 8), 4 and 2 that
    divides it, else 1 (int64: 1)."""
    if is_int(dtype):
        return 1
    for lanes in (8, 4, 2):
        if lanes <= limit and extent % lanes == 0:
            return lanes
    return 1
