"""Pin the rotary-embedding oracle (CPU only).

oracle.rope restates the reference's rotary angles and the q/k rotation of
Ouro's attention (vllm_rlt/models/ouro.py:39-75, 104-109).  It is checked
against the reference's own output bits (tests/golden/rotary_cpu.npz), against
the identity at position 0, and against an independent float64 evaluation
written as a complex multiplication.  Planted mistakes (a wrong sign in
rotate_half, swapped halves, angles from the wrong frequency) fail the pins.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import rope

GOLDEN = Path(__file__).resolve().parent / "golden" / "rotary_cpu.npz"
DTYPES = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}
BITS = {torch.bfloat16: torch.int16, torch.float16: torch.int16, torch.float32: torch.int32}


def golden_cases():
    data = np.load(GOLDEN)
    names = sorted({k.split("/")[0] for k in data.files})
    cases = {}
    for name in names:
        dtype = DTYPES[str(data[f"{name}/dtype"])]
        fields = {f: torch.from_numpy(data[f"{name}/{f}"]).view(dtype) for f in ("x", "cos", "sin", "out")}
        fields["positions"] = torch.from_numpy(data[f"{name}/positions"])
        fields["theta"] = float(data[f"{name}/theta"])
        fields["dtype"] = dtype
        cases[name] = fields
    return cases


CASES = golden_cases()


def same_bits(a: torch.Tensor, b: torch.Tensor) -> bool:
    return torch.equal(a.contiguous().view(BITS[a.dtype]), b.contiguous().view(BITS[b.dtype]))


@pytest.mark.parametrize("name", sorted(CASES))
def test_cos_sin_match_reference_bits(name):
    c = CASES[name]
    cos, sin = rope.rotary_cos_sin(c["positions"], c["x"].shape[-1], c["theta"], c["dtype"])
    assert same_bits(cos, c["cos"]) and same_bits(sin, c["sin"])


@pytest.mark.parametrize("name", sorted(CASES))
def test_rotation_matches_reference_bits(name):
    c = CASES[name]
    assert same_bits(rope.apply_rotary(c["x"], c["cos"], c["sin"]), c["out"])


@pytest.mark.parametrize("name", sorted(CASES))
def test_position_zero_is_identity(name):
    c = CASES[name]
    zero = c["positions"] == 0
    assert zero.any()
    assert same_bits(c["out"][zero], c["x"][zero])


def rotation_f64(x: torch.Tensor, positions: torch.Tensor, theta: float) -> np.ndarray:
    """(x_lo + i x_hi) * exp(i * pos * theta^(-2j/D)) in float64, halves re-split."""
    d = x.shape[-1]
    half = d // 2
    inv = 1.0 / theta ** (np.arange(0, d, 2, dtype=np.float64) / d)
    ang = positions.numpy().astype(np.float64)[:, None] * inv[None, :]
    z = x.double().numpy()
    w = (z[..., :half] + 1j * z[..., half:]) * np.exp(1j * ang)[:, None, :]
    return np.concatenate([w.real, w.imag], axis=-1)


@pytest.mark.parametrize("name", sorted(CASES))
def test_rotation_agrees_with_float64_complex_rotation(name):
    c = CASES[name]
    expect = rotation_f64(c["x"], c["positions"], c["theta"])
    got = c["out"].double().numpy()
    # cos/sin are rounded to the storage dtype and the angle is a float32
    # product, so the tolerance is a few storage ulps of |x| plus the float32
    # angle error at large positions.
    eps = {torch.bfloat16: 2**-8, torch.float16: 2**-11, torch.float32: 2**-23}[c["dtype"]]
    scale = np.abs(c["x"].double().numpy()).max()
    pos_err = float(c["positions"].max()) * 2**-24 * 2
    assert np.abs(got - expect).max() <= scale * (6 * eps + pos_err)


def test_planted_mistakes_fail_the_pins():
    c = CASES["bf16_ouro"]

    def bad_sign(x):
        first, second = x.chunk(2, dim=-1)
        return torch.cat((second, first), dim=-1)

    def swapped(x):
        first, second = x.chunk(2, dim=-1)
        return torch.cat((first, -second), dim=-1)

    for mistake in (bad_sign, swapped):
        out = c["x"] * c["cos"].unsqueeze(1) + mistake(c["x"]) * c["sin"].unsqueeze(1)
        assert not same_bits(out, c["out"])
    # Angles from the half-width frequency table (a plausible indexing slip).
    cos, _ = rope.rotary_cos_sin(c["positions"], c["x"].shape[-1] // 2, c["theta"], c["dtype"])
    assert not same_bits(torch.cat([cos, cos], dim=-1), c["cos"])


def test_rope_append_writes_rotated_k_and_plain_v():
    torch.manual_seed(0)
    nb, layers, page, hkv, d = 5, 2, 4, 2, 8
    kc = torch.zeros(nb, layers, page, hkv, d, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    q = torch.randn(3, 4, d).to(torch.bfloat16)
    k = torch.randn(3, hkv, d).to(torch.bfloat16)
    v = torch.randn(3, hkv, d).to(torch.bfloat16)
    cos, sin = rope.rotary_cos_sin(torch.tensor([0, 5, 9]), d, 10000.0, torch.bfloat16)
    q_rot = rope.rope_append(kc, vc, 1, [4, 0, 2], [3, 1, 0], q, k, v, cos, sin, n_rows=2)
    assert same_bits(q_rot, rope.apply_rotary(q, cos, sin))
    assert same_bits(kc[4, 1, 3], rope.apply_rotary(k, cos, sin)[0])
    assert same_bits(vc[0, 1, 1], v[1])
    assert not kc[2].any() and not vc[2].any()  # the padding row is not written
