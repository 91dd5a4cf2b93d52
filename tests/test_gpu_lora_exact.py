"""Exact LoRA results on every kernel path, rank tile by rank tile.

The base weight is zero (int4: q = 0 with scale 0; fp8: zero bytes with
unit channel scales), x and dy are one-hot token rows and A, B hold small
integers, so every output is a short sum of small multiples of 1/2: exact
in f32 and in bf16 whatever the summation order. y, t, dx, dA and dB must
then equal the integer closed form bit for bit. A rank chunk of 16 whose
matrix-core step was skipped, or an accumulator element read before its
last step landed, changes the elements that chunk contributes to, and the
test checks that the last chunk contributes to a large share of them.

Each case selects one kernel path of the library (256 CUs): the few-token
kernels (m <= 16), the split-depth GEMM with 192-row tiles (m = 256, forced
onto the large tiles), the tiled GEMM with 192-row and 256-row tiles
(m = 4096), and the mid-size tiles of 64 and 128 tokens (forced, with a
ragged token count), forward and backward. Ranks 16, 32, 33, 48 and 64
cover one to four rank chunks and a padded chunk.
"""

import numpy as np
import pytest
import torch

from gpu_helpers import gemm_path
from loractl_amd import _lib as L
from loractl_amd import device as D

pytestmark = pytest.mark.gpu

SCALING = 0.5
# (label, M, K, N, GEMM path)
PATHS = [
    ("few-token m=5", 5, 512, 768, "planned"),
    ("few-token m=16", 16, 3072, 3072, "planned"),
    ("few-token split forward m=9", 9, 4160, 520, "planned"),
    ("few-token whole-depth forward m=16", 16, 3072, 8192, "planned"),
    ("split-depth r192", 256, 3072, 3072, "large"),
    ("tiled r192 fwd / split bwd", 4096, 256, 3072, "large"),
    ("tiled r256", 4096, 4096, 4096, "large"),
    ("tiled, ragged tokens", 1100, 1024, 2048, "large"),
    ("mid 64-token tiles", 300, 3072, 3064, "mid64"),
    ("mid 128-token tiles", 300, 1088, 1032, "mid128"),
    ("mid 64-token tiles, depth ranges", 200, 3072, 2560, "mid64s"),
    ("mid 128-token tiles, depth ranges", 256, 2560, 9728, "mid128s"),
]
RANKS = [16, 32, 33, 48, 64]


def _closed_form(M, K, N, r):
    m = np.arange(M)
    km = (7 * m + 3) % K          # x[m] = e_km
    nm = (5 * m + 1) % N          # dy[m] = e_nm
    g = np.random.Generator(np.random.PCG64(M * 7919 + K * 31 + N + r))
    A = g.integers(-2, 3, (K, r)).astype(np.int64)              # [K, r] in -2..2
    B = g.integers(-1, 2, (r, N)).astype(np.int64)              # [r, N] in -1..1
    # twice the values (SCALING = 1/2), as integers
    t2 = A[km]                                                  # 2 t = A[km]
    y2 = t2 @ B                                                 # 2 y = (2 t) . B
    u2 = B[:, nm].T                                             # 2 u = B[:, nm]
    dx2 = u2 @ A.T                                              # 2 dx = u2 . A^T
    da2 = np.zeros((K, r), np.int64)
    np.add.at(da2, km, u2)                                      # 2 dA = x^T . (2 u)
    db2 = np.zeros((r, N), np.int64)
    np.add.at(db2.T, nm, t2)                                    # 2 dB = (2 t)^T . dy
    return dict(km=km, nm=nm, A=A, B=B, t=t2 / 2, y=y2 / 2, dx=dx2 / 2, da=da2 / 2, db=db2 / 2)


def _weight(fmt, N, K, dev):
    if fmt == "int4":
        return D.quantize_int4(torch.zeros((N, K), dtype=torch.float32, device=dev), 64)
    return D.PackedWeight(L.LRQ_FMT_FP8, N, K, torch.zeros((N, K), dtype=torch.uint8, device=dev),
                          torch.ones((N,), dtype=torch.float32, device=dev), per_channel=True)


def _exact(name, got, ref):
    g = got.float().cpu().numpy().astype(np.float64)
    bad = np.argwhere(g != ref)
    assert bad.size == 0, (f"{name}: {len(bad)} of {ref.size} elements differ; first at {tuple(bad[0])}: "
                           f"got {g[tuple(bad[0])]}, want {ref[tuple(bad[0])]}")


@pytest.mark.parametrize("fmt", ["int4", "fp8"])
@pytest.mark.parametrize("r", RANKS)
@pytest.mark.parametrize("label,M,K,N,path", PATHS, ids=[p[0] for p in PATHS])
def test_lora_exact_per_rank_chunk(cuda, label, M, K, N, path, r, fmt):
    print(f"[exact] {label} M={M} K={K} N={N} r={r} {fmt} {path}", flush=True)
    cf = _closed_form(M, K, N, r)
    # the test's power: the last rank chunk (16 wide, possibly padded)
    # changes a large share of the outputs, so skipping its step cannot go unseen
    j0 = (r - 1) // 16 * 16
    for part in (cf["t"][:, j0:] @ cf["B"][j0:, :], (cf["B"][j0:, cf["nm"]].T / 2) @ cf["A"][:, j0:].T):
        assert (part != 0).mean() > 0.4
    x = torch.zeros((M, K), dtype=torch.bfloat16, device=cuda)
    x[torch.arange(M), torch.from_numpy(cf["km"]).to(cuda)] = 1
    dy = torch.zeros((M, N), dtype=torch.bfloat16, device=cuda)
    dy[torch.arange(M), torch.from_numpy(cf["nm"]).to(cuda)] = 1
    a = torch.from_numpy(cf["A"]).to(cuda).to(torch.bfloat16).contiguous()
    b = torch.from_numpy(cf["B"]).to(cuda).to(torch.bfloat16).contiguous()
    wq = _weight(fmt, N, K, cuda)
    with gemm_path(path):
        y, t = D.lora_fwd(x, wq, a, b, SCALING)
        dx, da, db = D.lora_bwd(x, dy, wq, a, b, SCALING, t)
        torch.cuda.synchronize()
    _exact("t", t, cf["t"])
    _exact("y", y, cf["y"])
    _exact("dx", dx, cf["dx"])
    _exact("dA", da, cf["da"])
    _exact("dB", db, cf["db"])
