"""Helpers of the GPU parity tests: seeded inputs representable in the kernel
dtype, moved to the device, plus the fp32 copies the oracle runs on."""
import numpy as np
import torch

from oracle import saga_oracle as O

TORCH_DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def round_to(x: np.ndarray, dt: str) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    if dt == "bf16":
        return O.round_bf16(x)
    if dt == "f16":
        return x.astype(np.float16).astype(np.float32)
    return x


def dev(x: np.ndarray, dt: str = "f32") -> torch.Tensor:
    """float32 numpy array (already representable in dt) -> device tensor of dt."""
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to("cuda").to(TORCH_DT[dt])


def randn(rng, shape, dt="f32", scale=1.0):
    x = round_to(rng.standard_normal(shape, dtype=np.float32) * np.float32(scale), dt)
    return x, dev(x, dt)


def host(t: torch.Tensor) -> np.ndarray:
    return t.detach().to(torch.float32).cpu().numpy()


def qkv(rng, b, q_h, k_h, v_h, d, L, dt, qscale=1.0, outliers=0.0):
    """Queries, keys, values ~ N(0,1); `outliers`: fraction of key rows x8."""
    q, qd = randn(rng, (b, q_h, 1, d), dt, qscale)
    kf = rng.standard_normal((b, k_h, L, d), dtype=np.float32)
    if outliers:
        rows = rng.random((b, k_h, L)) < outliers
        kf[rows] *= np.float32(8.0)
    k = round_to(kf, dt)
    v, vd = randn(rng, (b, v_h, L, d), dt)
    return (q, k, v), (qd, dev(k, dt), vd)
