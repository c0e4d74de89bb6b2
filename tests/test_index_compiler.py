"""The generated kernels' index arithmetic, pinned by brute force.

``Kernel.div``/``Kernel.mod``/``Kernel.unflatten`` fold exactly when bounds allow and otherwise declare
opaque atoms. Every simplified form is evaluated here over *all* values of its atoms and compared with
plain integer division and remainder, for random affine forms and for the address maps that views,
reshapes and transposes produce.
"""

import itertools
import random

import pytest

from chroma_amd._src.codegen.kernel import Aff, Atom, Kernel
from chroma_amd._src.value import contiguous_strides


def evaluate(kernel: Kernel, aff: Aff, env: dict) -> int:
    total = aff.const
    for atom, coef in aff.terms:
        if atom.name not in env:
            op, operand, constant = kernel.definitions[atom.name]
            inner = evaluate(kernel, operand, env)
            env[atom.name] = inner // constant if op == "div" else inner % constant
        total += coef * env[atom.name]
    return total


def all_values(atoms):
    for values in itertools.product(*(range(a.hi + 1) for a in atoms)):
        yield dict(zip((a.name for a in atoms), values))


@pytest.mark.parametrize("seed", range(40))
def test_div_mod_of_random_affine_forms(seed):
    rng = random.Random(seed)
    atoms = [Atom(f"x{i}", rng.randint(1, 6)) for i in range(rng.randint(1, 3))]
    aff = Aff([(a, rng.choice([1, 2, 3, 4, 6, 8, 12, 16])) for a in atoms], rng.randint(0, 20))
    for constant in (1, 2, 3, 4, 5, 8, 16, 24):
        kernel = Kernel()
        quotient, remainder = kernel.div(aff, constant), kernel.mod(aff, constant)
        for env in all_values(atoms):
            value = evaluate(kernel, aff, dict(env))
            assert evaluate(kernel, quotient, dict(env)) == value // constant
            assert evaluate(kernel, remainder, dict(env)) == value % constant
            assert 0 <= evaluate(kernel, quotient, dict(env)) <= quotient.hi()
            assert 0 <= evaluate(kernel, remainder, dict(env)) <= remainder.hi()


def test_head_major_addresses_fold_without_an_opaque_division():
    """(4096 * token + 64 * head + j) / 512 and % 512 for j < 32 (a rotary half of a head of 64 inside a
    [tokens, 8, 8, 64] view): the head term is split as 512 * (head / 8) + 64 * (head % 8), so the
    quotient is 8 * token + head / 8 and no division of the whole address is declared; correct for every
    value."""
    kernel = Kernel()
    token, head, j = Atom("t", 3), Atom("h", 63), Atom("j", 31)
    aff = Aff(((token, 4096), (head, 64), (j, 1)), 0)
    quotient, remainder = kernel.div(aff, 512), kernel.mod(aff, 512)
    declared = [kernel.definitions[a.name] for a, _ in quotient.terms + remainder.terms if a.name in kernel.definitions]
    assert declared and all(operand != aff for _, operand, _ in declared)  # only head / 8 and head % 8
    assert quotient.coefficient(token) == 8 and quotient.coefficient(j) == 0
    for env in all_values([token, head, j]):
        value = evaluate(kernel, aff, dict(env))
        assert evaluate(kernel, quotient, dict(env)) == value // 512
        assert evaluate(kernel, remainder, dict(env)) == value % 512


@pytest.mark.parametrize("seed", range(30))
def test_view_addresses_decode_to_the_right_coordinates(seed):
    """A permuted / sliced / broadcast view of a contiguous source, read through flat-index decoding."""
    rng = random.Random(1000 + seed)
    source = [rng.randint(1, 4) for _ in range(rng.randint(1, 3))]
    order = list(range(len(source)))
    rng.shuffle(order)
    view_shape = [source[d] for d in order]
    strides = [contiguous_strides(source)[d] for d in order]
    kernel = Kernel()
    coords_atoms = [Atom(f"c{i}", s - 1) for i, s in enumerate(view_shape)]
    coords = [Aff.of(a) for a in coords_atoms]
    flat = Aff((), 0)
    for coord, stride in zip(coords, strides):
        flat = flat + coord.scale(stride)
    decoded = kernel.unflatten(flat, source)
    for env in all_values(coords_atoms):
        values = [env[a.name] for a in coords_atoms]
        expected_source = [0] * len(source)
        for axis, value in zip(order, values):
            expected_source[axis] = value
        assert [evaluate(kernel, d, dict(env)) for d in decoded] == expected_source


@pytest.mark.parametrize("shapes", [((8, 128), (8, 8, 16)), ((6, 4), (24,)), ((2, 3, 4), (4, 6)), ((5, 7), (35,)), ((12,), (3, 2, 2))])
def test_reshape_roundtrip(shapes):
    old, new = shapes
    kernel = Kernel()
    atoms = [Atom(f"c{i}", s - 1) for i, s in enumerate(new)]
    flat = Kernel.flatten([Aff.of(a) for a in atoms], new)
    decoded = kernel.unflatten(flat, old)
    for env in all_values(atoms):
        linear = sum(env[a.name] * s for a, s in zip(atoms, contiguous_strides(new)))
        expected = [linear // s % n for s, n in zip(contiguous_strides(old), old)]
        assert [evaluate(kernel, d, dict(env)) for d in decoded] == expected


def test_bounds_proof_rejects_an_access_past_the_buffer():
    kernel = Kernel()
    slot = kernel.slot("buffer", __import__("torch").float32, extent=16)
    atom = Atom("i", 15)
    kernel.check_bounds(slot, Aff.of(atom))
    with pytest.raises(AssertionError, match="may exceed"):
        kernel.check_bounds(slot, Aff.of(atom) + 1)
