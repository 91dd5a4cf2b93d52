"""Seeded inputs and comparisons shared by the GPU parity tests."""

import contextlib

import numpy as np
import torch

import oracle as O

TOL_REL = 1e-2     # rel_deviation (peak-normalized, accuracy.rs:107) for bf16 outputs
TOL_COS = 0.999    # cosine similarity floor


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def case_inputs(M, K, N, r, seed=0, b_sigma=1e-2):
    """W ~ N(0, 0.02) f32 [N,K]; X, dY ~ N(0,1) and A ~ U(+-1/sqrt(K)), B ~ N(0, b_sigma)
    rounded to bf16 (the values both sides see)."""
    w = (rng(seed).standard_normal((N, K)) * 0.02).astype(np.float32)
    x = O.bf16_round(rng(seed + 1).standard_normal((M, K)).astype(np.float32))
    a = O.bf16_round(rng(seed + 2).uniform(-1 / np.sqrt(K), 1 / np.sqrt(K), (K, max(r, 1))).astype(np.float32))
    b = O.bf16_round((rng(seed + 3).standard_normal((max(r, 1), N)) * b_sigma).astype(np.float32))
    dy = O.bf16_round(rng(seed + 4).standard_normal((M, N)).astype(np.float32))
    return w, x, a, b, dy


def to_dev(v, dev, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(v)).to(dev).to(dtype)


def check(name, got, ref, tol_rel=TOL_REL, tol_cos=TOL_COS):
    g = got.detach().float().cpu().numpy() if isinstance(got, torch.Tensor) else np.asarray(got, np.float32)
    rel = O.rel_deviation(g, ref)
    cos = O.cosine(g, ref) if np.abs(ref).max() > 0 else (1.0 if not np.abs(g).max() else 0.0)
    assert rel <= tol_rel and cos >= tol_cos, f"{name}: rel_dev={rel:.3e} cos={cos:.6f}"
    return rel, cos


@contextlib.contextmanager
def gemm_path(path):
    """Run the block with the fused products of m > 16 tokens forced onto one
    kernel path ("planned", "large", "mid64", "mid128", "mid64s", "mid128s")."""
    from loractl_amd import device as D

    D.debug_gemm_path(path)
    try:
        yield
    finally:
        D.debug_gemm_path("planned")
