"""Writes the committed HiF8 fixtures from the CPU oracle (oracle/hif8_ref.py).

The reference cannot run here (its only qdq kernel is Ascend C and its Python
path imports an aarch64 extension), so these vectors come from the oracle,
whose every function is pinned by the closed-form tests in tests/test_oracle.py.
They give the GPU tests exact expectations without recomputation and pin the
oracle itself across machines.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import hif8_ref as R  # noqa: E402


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def exhaustive():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    xf = R.bf16_to_f32(bits)
    npu = R.f32_to_bf16(R.quant_hif8_npu(xf))
    torch_ = R.f32_to_bf16(R.quant_hif8_torch(xf))
    codes = R.encode_npu(xf)        # NaN -> the -Inf code: the NPU qdq of NaN is -Inf
    np.savez_compressed(os.path.join(HERE, "hif8_bf16_exhaustive.npz"), npu_qdq=npu, torch_qdq=torch_,
                        codes=codes, decode=R.decode_table())


def scales():
    a = np.arange(32768, dtype=np.uint16)
    s15 = np.array([R.hif8_scale_bf16(int(v), 15.0) for v in a], np.uint16)
    s224 = np.array([R.hif8_scale_bf16(int(v), 224.0) for v in a], np.uint16)
    np.savez_compressed(os.path.join(HERE, "hif8_scale_bf16.npz"), amax=a, scale15=s15, scale224=s224)


def config1():
    x = R.c1_input(0)
    xq_npu, s_bits = R.quant_bf16(x, 15.0, "npu")
    xq_torch, _ = R.quant_bf16(x, 15.0, "torch")
    codes, s2 = R.codes_bf16(x, 15.0)
    assert s2 == s_bits
    amax = R.absmax_bf16(x)
    rng = np.random.default_rng(1234)
    idx = np.sort(rng.choice(x.size, 4096, replace=False))
    diff = np.nonzero(xq_npu.ravel() != xq_torch.ravel())[0]
    idx = np.unique(np.concatenate([idx, diff]))
    np.savez_compressed(os.path.join(HERE, "c1_samples.npz"), idx=idx, x=x.ravel()[idx], codes=codes.ravel()[idx],
                        xq_npu=xq_npu.ravel()[idx], xq_torch=xq_torch.ravel()[idx])
    meta = {
        "recipe": "randn(4096,5120, seed 0)*0.02; randperm(n)[:n//1000] *= 50; bf16",
        "amax_bits": int(amax), "scale_bits": int(s_bits),
        "sha256_codes": sha(codes), "sha256_xq_npu": sha(xq_npu), "sha256_xq_torch": sha(xq_torch),
        "n_semantics_differ": int(diff.size),
    }
    with open(os.path.join(HERE, "c1_digest.json"), "w") as f:
        json.dump(meta, f, indent=1)


if __name__ == "__main__":
    R.build_lib()
    exhaustive()
    scales()
    config1()
    print("fixtures written to", HERE)
