"""The oracle's DiT block norm and AdaSingle modulation (orc_ada_in,
orc_ada_out; the block graph's modulation inputs, seedvr2_dit.cpp:441-448,
734-738), pinned independently of its own formula: torch's float64 rms_norm,
the unit-RMS and scale-invariance properties of the norm, per-sample constants
that identify each row's sample, and the exact identities of the gate."""
import numpy as np
import pytest
import torch

import oracle

DIM = 96
ROWS = [5, 1, 9]


def _x(seed, rows=sum(ROWS), dim=DIM):
    g = np.random.default_rng(seed)
    return (g.standard_normal((rows, dim)) * g.uniform(0.1, 10, (rows, 1))).astype(np.float32)


def _vec(seed, batch, dim=DIM, std=1.0, mean=0.0):
    g = np.random.default_rng(seed)
    return (mean + std * g.standard_normal((batch, dim))).astype(np.float32)


def _sample_of_rows(counts):
    return np.repeat(np.arange(len(counts)), counts)


def test_ada_in_matches_torch_rms_norm():
    x = _x(1)
    b = len(ROWS)
    sa, ca = _vec(2, b), _vec(3, b, mean=1.0)
    sb, cb = _vec(4, 1)[0], _vec(5, 1, std=0.1)[0]
    got = oracle.ada_in(x, ROWS, sa, ca, sb, cb, eps=1e-5)
    xt = torch.from_numpy(x).double()
    n = torch.nn.functional.rms_norm(xt, (DIM,), eps=1e-5)
    s = _sample_of_rows(ROWS)
    ref = n * torch.from_numpy(ca[s] + cb).double() + torch.from_numpy(sa[s] + sb).double()
    np.testing.assert_allclose(got, ref.numpy(), rtol=2e-6, atol=2e-6)


def test_ada_in_unit_rms_at_identity_modulation():
    x = _x(6)
    b = len(ROWS)
    eps = 1e-5
    got = oracle.ada_in(x, ROWS, np.zeros((b, DIM)), np.ones((b, DIM)), eps=eps)
    ms = np.mean(x.astype(np.float64) ** 2, axis=1)
    np.testing.assert_allclose(np.mean(got.astype(np.float64) ** 2, axis=1), ms / (ms + eps),
                               rtol=1e-5)


def test_ada_in_is_scale_invariant_without_eps():
    x = _x(7)
    b = len(ROWS)
    sa, ca = _vec(8, b), _vec(9, b)
    a = oracle.ada_in(x, ROWS, sa, ca, eps=0.0)
    c = oracle.ada_in(x * np.float32(4.0), ROWS, sa, ca, eps=0.0)   # exact scaling by 4
    np.testing.assert_array_equal(a, c)


def test_ada_in_rows_take_their_sample_vectors():
    x = _x(10)
    b = len(ROWS)
    # scale 0 leaves only the shift: sample k's rows are its constant k + 1
    shift = np.repeat(np.arange(1, b + 1, dtype=np.float32)[:, None], DIM, 1)
    got = oracle.ada_in(x, ROWS, shift, np.zeros((b, DIM)), shift_b=np.full(DIM, 0.5))
    np.testing.assert_array_equal(got, (_sample_of_rows(ROWS) + 1.5)[:, None] * np.ones(DIM))


def test_ada_out_gate_identities():
    x, y = _x(11), _x(12)
    b = len(ROWS)
    np.testing.assert_array_equal(oracle.ada_out(x, y, ROWS, np.zeros((b, DIM))), x)
    np.testing.assert_array_equal(oracle.ada_out(x, y, ROWS, np.ones((b, DIM))),
                                  (x + y).astype(np.float32))
    # gate_a + gate_b: 0.75 + 0.25 = 1 exactly
    np.testing.assert_array_equal(
        oracle.ada_out(x, y, ROWS, np.full((b, DIM), 0.75), np.full(DIM, 0.25)), x + y)


def test_ada_out_rows_take_their_sample_gates():
    b = len(ROWS)
    x = np.zeros((sum(ROWS), DIM), np.float32)
    y = np.ones_like(x)
    gates = np.repeat(np.arange(b, dtype=np.float32)[:, None] * 2, DIM, 1)
    got = oracle.ada_out(x, y, ROWS, gates)
    np.testing.assert_array_equal(got[:, 0], _sample_of_rows(ROWS) * 2.0)


@pytest.mark.parametrize("counts", [[0, 4], [3, 0, 2]])
def test_empty_samples_take_no_rows(counts):
    x = _x(13, rows=sum(counts))
    b = len(counts)
    shift = np.repeat(np.arange(b, dtype=np.float32)[:, None], DIM, 1)
    got = oracle.ada_in(x, counts, shift, np.zeros((b, DIM)))
    np.testing.assert_array_equal(got[:, 0], _sample_of_rows(counts).astype(np.float32))
