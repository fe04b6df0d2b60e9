"""GPU test helpers: device tensors from numpy and the parity metrics."""
import numpy as np
import torch

from ferrisres_amd import synth

DEV = "cuda:0"


def dev_u32(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).to(DEV)


def dev_f32(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(DEV)


def dev_bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)).to(DEV).view(torch.bfloat16)


def host(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        return synth.bf16_bits_to_f32(t.view(torch.int16).cpu().numpy().view(np.uint16))
    return t.cpu().numpy()


def assert_close_f32(y: np.ndarray, ref: np.ndarray, tol: float = 1e-3):
    """Elementwise |y-ref| <= tol * max(|ref|, rms(ref)) and normwise
    ||y-ref||_inf <= tol * ||ref||_inf."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    assert y.shape == ref.shape, (y.shape, ref.shape)
    assert np.isfinite(y).all()
    rms = np.sqrt((ref ** 2).mean()) if ref.size else 0.0
    err = np.abs(y - ref)
    bound = tol * np.maximum(np.abs(ref), rms)
    bad = err > bound
    assert not bad.any(), f"{bad.sum()} elements out of tolerance; worst rel {(err / np.maximum(bound, 1e-30)).max() * tol:.3g}"
    assert err.max() <= tol * np.abs(ref).max() + 1e-30


def assert_bf16_within_1ulp(y_bits: np.ndarray, ref: np.ndarray, tol: float = 1e-3):
    """bf16 outputs within 1 ulp of bf16(ref). Where |ref| is below the noise
    floor of the f32 criterion (tol * rms(ref)) the reference value itself is
    summation-order noise, so there the f32 criterion |y - ref| <= tol * rms
    applies instead."""
    ref = np.asarray(ref, np.float32)
    r = synth.f32_to_bf16_bits(ref).astype(np.int32)
    y = np.asarray(y_bits, np.uint16).astype(np.int32)

    def order(b):  # ordered integer view of bf16 (sign-magnitude)
        return np.where(b & 0x8000, -(b & 0x7FFF), b & 0x7FFF)
    ulps = np.abs(order(y) - order(r))
    rms = float(np.sqrt((ref.astype(np.float64) ** 2).mean())) if ref.size else 0.0
    yf = synth.bf16_bits_to_f32(np.asarray(y_bits, np.uint16)).astype(np.float64)
    floor_ok = np.abs(yf - ref) <= tol * rms
    bad = (ulps > 1) & ~floor_ok
    assert not bad.any(), f"{bad.sum()} bf16 outputs more than 1 ulp off above the noise floor (max {ulps[bad].max()} ulp)"
