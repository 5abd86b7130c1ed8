"""CPU tests of the product's host-side pieces (no GPU work):

* the C-ABI library loads and exports every symbol include/hif8_mi355x.h declares,
  and the Python binding declares the same set;
* argument validation returns the documented status codes before any launch;
* the kernels' shared HiF8 arithmetic (hif8_common.h), built for the host,
  matches the oracle for every bf16 input, random fp32 inputs, every code, and
  the LDS encode table.
"""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hif8_mi355x.h")


def header_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(hif8_\w+)\s*\(", src)))


def test_library_exports_every_declared_symbol(pkg):
    L = pkg._lib.load()
    names = header_functions()
    assert len(names) >= 12
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(pkg._lib.SIGNATURES), "binding and header disagree"
    out = subprocess.run(["nm", "-D", "--defined-only", pkg._lib.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (hif8_\w+)", out))
    assert set(names) <= exported


def test_status_codes_without_gpu(pkg):
    L = pkg._lib.load()
    assert L.hif8_state_size() % 256 == 0
    assert L.hif8_strerror(0) == b"ok"
    fake = 0x100000      # aligned, never dereferenced: validation fails first
    odd = 0x100001
    assert L.hif8_state_init(None, None) == -1
    assert L.hif8_absmax_scale(None, 0, 16, 15.0, fake, None) == -1
    assert L.hif8_absmax_scale(fake, 0, 0, 15.0, fake, None) == -1
    assert L.hif8_absmax_scale(fake, 7, 16, 15.0, fake, None) == -1
    assert L.hif8_absmax_scale(odd, 0, 16, 15.0, fake, None) == -3
    assert L.hif8_encode(fake, 0, 16, None, fake, None) == -1
    assert L.hif8_fake_quant(fake, 0, 16, fake, fake, 5, None) == -1
    assert L.hif8_fake_quant(fake, 0, 16, fake, odd, 0, None) == -3
    assert L.hif8_quant_bf16(None, fake, 16, 0, None) == -1
    assert L.hif8_decode(fake, -1, fake, 0, fake, None) == -1
    # linear: missing pointers, K % 64, N % 8, alignment
    args = dict(a=fake, w=fake, wst=fake, b=None, y=fake, M=128, N=256, K=512)

    def lin(**kw):
        a = {**args, **kw}
        return L.hif8_linear_fwd(a["a"], a["w"], a["wst"], a["b"], a["y"], a["M"], a["N"], a["K"], None)
    assert lin(a=None) == -1
    assert lin(wst=None) == -1
    assert lin(M=0) == -1
    assert lin(K=100) == -2
    assert lin(N=100) == -2
    assert lin(y=odd) == -3
    assert lin(b=fake + 2) == -3
    assert lin(K=1 << 22) == -2          # bf16 activations: K < 2^22 (32-bit buffer offsets)
    # grouped linear: group count, shapes of the groups, alignment
    P = ctypes.c_void_p
    I64 = ctypes.c_int64

    def grp(ns, sts=None, ys=None, a=fake, w=fake, b=None, K=512):
        g = len(ns)
        sts = (P * g)(*([fake] * g if sts is None else sts))
        ys = (P * g)(*([fake] * g if ys is None else ys))
        return L.hif8_linear_fwd_grouped(a, w, sts, b, ys, (I64 * g)(*ns), g, 128, K, None)
    assert grp([256, 256, 264], a=None) == -1
    assert L.hif8_linear_fwd_grouped(fake, fake, None, None, None, None, 0, 128, 512, None) == -1
    assert grp([256] * 9) == -2                        # at most 8 groups
    assert grp([264, 256]) == -2                       # all but the last a multiple of 256
    assert grp([256, 260]) == -2                       # the last a multiple of 8
    assert grp([256, 256], K=100) == -2
    assert grp([256, 256], sts=[fake, None]) == -1
    assert grp([256, 256], ys=[fake, odd]) == -3
    assert grp([256, 256], b=fake + 2) == -3
    # token-major wgrad: pointers, sizes, n_out and k_in % 8, the 32-bit offset limit, alignment
    # (all checked before any device call)
    assert L.hif8_linear_wgrad(None, fake, fake, 1024, 256, 256, None, 0, None) == -1
    assert L.hif8_linear_wgrad(fake, fake, fake, 0, 256, 256, None, 0, None) == -1
    assert L.hif8_linear_wgrad(fake, fake, fake, 1024, 260, 256, None, 0, None) == -2
    assert L.hif8_linear_wgrad(fake, fake, fake, 1024, 256, 100, None, 0, None) == -2
    assert L.hif8_linear_wgrad(fake, fake, fake, 1 << 23, 256, 256, None, 0, None) == -2   # 4 GB of grad_q
    assert L.hif8_linear_wgrad(fake, fake, fake, 1 << 20, 2048, 16, None, 0, None) == -2   # (2^20 + 128) * 4 KB
    assert L.hif8_linear_wgrad(fake, odd, fake, 1024, 256, 256, None, 0, None) == -3
    # split-tail GEMM: pointers and the shapes of hif8_linear_fwd_wq
    assert L.hif8_linear_fwd_wq_split(None, fake, None, fake, 128, 256, 512, None, 0, None) == -1
    assert L.hif8_linear_fwd_wq_split(fake, fake, None, fake, 128, 256, 100, None, 0, None) == -2
    assert L.hif8_linear_fwd_wq_split(fake, fake, None, odd, 128, 256, 512, None, 0, None) == -3
    assert L.hif8_linear_split_workspace_bytes(0, 256, 512) == 0
    # attention: pointers, sizes, head dim 128, strides, the 32-bit key offsets, the state's dtype,
    # alignment (all checked before any device call)
    def att(q=fake, out=fake, B=2, nq=300, nkv=200, H=4, D=128, rs=(512,) * 4, bs=(512 * 300,) * 4,
            idx=None, idx_bs=0, cnt=None, scale=0.088, st=None, st_dt=2, smax=15.0):
        return L.hif8_attention_fwd(q, fake, fake, out, B, nq, nkv, H, D, (I64 * 4)(*rs), (I64 * 4)(*bs), idx, idx_bs,
                                    cnt, scale, st, st_dt, smax, None)
    assert att(q=None) == -1
    assert att(nkv=0) == -1
    assert att(scale=0.0) == -1
    assert att(idx=fake) == -1                          # a key list needs its counts
    assert att(st=fake, st_dt=1) == -1                  # the o state: bf16 or bf16-as-fp32 rules
    assert att(D=64) == -2
    assert att(rs=(256, 512, 512, 512)) == -2           # row stride below heads * 128
    assert att(rs=(516, 512, 512, 512)) == -2           # row stride not a multiple of 8
    assert att(nkv=(1 << 20) + 1, rs=(512, 1024, 512, 512)) == -2   # 2 GB of key rows: 32-bit offsets
    assert att(nkv=2, rs=(512, 1 << 23, 512, 512)) == -2      # key row stride of 16 MB: 24-bit products
    assert att(out=odd) == -3
    assert att(idx=fake + 2, idx_bs=200, cnt=fake) == -3
    # modulated LayerNorm: dim % 8, dim <= 8192, alignment of x and of the row statistics
    assert L.hif8_modln_amax(None, None, None, 4, 5120, 4, 1e-6, fake, 15.0, fake, None) == -1
    assert L.hif8_modln_amax(fake, None, None, 0, 5120, 4, 1e-6, fake, 15.0, fake, None) == -1
    assert L.hif8_modln_amax(fake, None, None, 4, 5120, 0, 1e-6, fake, 15.0, fake, None) == -1
    assert L.hif8_modln_amax(fake, None, None, 4, 100, 4, 1e-6, fake, 15.0, fake, None) == -2
    assert L.hif8_modln_amax(fake, None, None, 4, 8200, 4, 1e-6, fake, 15.0, fake, None) == -2
    # the allocation-free producer: its static workspace bounds the rows, checked before any work
    assert L.hif8_modln_quant_static(fake, None, None, 131073, 5120, 131073, 1e-6, 15.0, 0, fake, None) == -5
    assert L.hif8_modln_quant_static(fake, None, None, 4, 5120, 4, 1e-6, 15.0, 7, fake, None) == -1
    assert L.hif8_modln_quant_static(fake, None, None, 4, 100, 4, 1e-6, 15.0, 0, fake, None) == -2
    assert L.hif8_modln_quant_static(fake, None, None, 4, 5120, 4, 1e-6, 15.0, 0, odd, None) == -3
    assert b"static workspace" in L.hif8_strerror(-5)
    assert L.hif8_modln_amax(odd, None, None, 4, 5120, 4, 1e-6, fake, 15.0, fake, None) == -3
    assert L.hif8_modln_amax(fake, odd, None, 4, 5120, 4, 1e-6, fake, 15.0, fake, None) == -3
    assert L.hif8_modln_amax(fake, None, None, 4, 5120, 4, 1e-6, fake + 4, 15.0, fake, None) == -3
    assert L.hif8_modln_fake_quant(fake, None, None, 4, 5120, 4, fake, fake, 0, None, None, None) == -1
    assert L.hif8_modln_fake_quant(fake, None, None, 4, 5120, 4, fake, fake, 9, fake, None, None) == -1
    assert L.hif8_modln_fake_quant(fake, None, None, 4, 5120, 4, fake, fake, 0, odd, None, None) == -3
    assert L.hif8_modln_fake_quant(fake, None, None, 4, 5120, 4, fake, fake, 0, fake, odd, None) == -3
    # GELU: the library's GELU and the GELU quantisation pass (pointers, sizes, semantics, alignment)
    assert L.hif8_gelu_bf16(None, fake, 16, None) == -1
    assert L.hif8_gelu_bf16(fake, fake, 0, None) == -1
    assert L.hif8_gelu_bf16(odd, fake, 16, None) == -3
    assert L.hif8_gelu_fake_quant(fake, 16, None, 15.0, fake, 0, None) == -1
    assert L.hif8_gelu_fake_quant(fake, 16, fake, 15.0, fake, 2, None) == -1      # NPU or torch only
    assert L.hif8_gelu_fake_quant(fake, 16, fake, 15.0, odd, 0, None) == -3
    # fp16 qdq: semantics 0, 1 and 3 (the fp16 torch route); any alignment
    assert L.hif8_quant_f16(None, fake, 16, 0, None) == -1
    assert L.hif8_quant_f16(fake, fake, 0, 3, None) == -1
    assert L.hif8_quant_f16(fake, fake, 16, 2, None) == -1
    # the fp32 GEMM and the zero padding: pointers, sizes, dtypes, strides, element size
    assert L.hif8_gemm_f32(None, 0, fake, 0, fake, 1, 4, 4, 4, 4, 1, 4, 1, None) == -1
    assert L.hif8_gemm_f32(fake, 0, fake, 0, fake, 1, 0, 4, 4, 4, 1, 4, 1, None) == -1
    assert L.hif8_gemm_f32(fake, 2, fake, 0, fake, 1, 4, 4, 4, 4, 1, 4, 1, None) == -1
    assert L.hif8_gemm_f32(fake, 0, fake, 0, fake, 1, 4, 4, 4, -4, 1, 4, 1, None) == -1
    assert L.hif8_gemm_f32(fake, 0, fake, 0, fake, 1, 64 * 65536, 4, 4, 4, 1, 4, 1, None) == -2
    assert L.hif8_pad_2d(None, 4, 4, fake, 8, 8, 2, None) == -1
    assert L.hif8_pad_2d(fake, 4, 4, fake, 0, 8, 2, None) == -1
    assert L.hif8_pad_2d(fake, 4, 4, fake, 8, 8, 3, None) == -1


def test_gemm_route_rule(pkg):
    """HIF8Linear's route for bf16 activations: decode-once from 8192 rows, or from 24576 rows
    when the reduction depth is at most 2048; GEMM_ROUTE forces either route."""
    hl = pkg.hif8_linear
    assert hl.GEMM_ROUTE == "auto"
    assert not hl.decode_once(8191, 5120) and hl.decode_once(8192, 5120)
    assert not hl.decode_once(24575, 1536) and hl.decode_once(24576, 1536)
    assert not hl.decode_once(8192, 2048) and hl.decode_once(8192, 2049)
    assert hl.decode_once(32760, 1536) and hl.decode_once(75600, 13824)
    old = hl.GEMM_ROUTE
    try:
        hl.GEMM_ROUTE = "fused"
        assert not hl.decode_once(75600, 5120)
        hl.GEMM_ROUTE = "decode_once"
        assert hl.decode_once(16, 64)
        hl.GEMM_ROUTE = "other"
        with pytest.raises(ValueError):
            hl.decode_once(16, 64)
    finally:
        hl.GEMM_ROUTE = old


def test_python_layer_refuses_cpu_tensors(pkg):
    torch = pytest.importorskip("torch")
    x = torch.zeros(16, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        pkg.quant_dequant_float(x, pkg.QType("hif8"))
    assert pkg.quant_dequant_float(x, pkg.QType("bf16")) is x
    # the attention kernel: GPU bf16 [B, N, H, 128] only, and no autograd
    q = torch.zeros(1, 4, 1, 128, dtype=torch.bfloat16)
    assert not pkg.attention_fwd_ok(q, q, q)
    with pytest.raises(ValueError):
        pkg.attention_fwd(q, q, q)
    with pytest.raises(RuntimeError):
        pkg.attention_fwd(q.clone().requires_grad_(True), q, q)
    with pytest.raises(ValueError):
        pkg.key_list(torch.ones(2, 3))          # not a bool mask


@pytest.fixture(scope="module")
def hostlib(tmp_path_factory):
    out = tmp_path_factory.mktemp("hostchk") / "libhostchk.so"
    src = os.path.join(ROOT, "tests", "host_encoder_check.cpp")
    subprocess.run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", src, "-o", str(out)], check=True)
    L = ctypes.CDLL(str(out))
    p = ctypes.c_void_p
    L.chk_encode_bits.argtypes = [p, p, ctypes.c_int64]
    L.chk_decode_bits.argtypes = [p]
    L.chk_table.argtypes = [p, p, p]
    L.chk_table.restype = ctypes.c_int64
    return L


def _enc(L, bits32):
    bits32 = np.ascontiguousarray(bits32, np.uint32)
    c = np.empty(bits32.shape, np.uint8)
    L.chk_encode_bits(bits32.ctypes.data, c.ctypes.data, bits32.size)
    return c


def test_device_encoder_matches_oracle_every_bf16(hostlib, R):
    b = np.arange(65536, dtype=np.uint32)
    xf = (b << 16).view(np.float32)
    fin = ~np.isnan(xf)
    got = _enc(hostlib, b << 16)
    assert np.array_equal(got, R.encode_npu(xf))        # NaN included
    assert np.all(got[~fin] == 0xEF)                     # the -Inf code, as the Ascend kernel's NaN output


def test_device_encoder_matches_oracle_random_fp32(hostlib, R):
    rng = np.random.default_rng(11)
    u = rng.integers(0, 2 ** 32, 1_000_000, dtype=np.uint64).astype(np.uint32)
    # concentrate half of them on the HiF8 range
    e = rng.integers(-26, 18, 500_000)
    v = (np.ldexp(rng.random(500_000) + 1, e) * rng.choice([-1, 1], 500_000)).astype(np.float32)
    u = np.concatenate([u, v.view(np.uint32)])
    xf = u.view(np.float32)
    assert np.array_equal(_enc(hostlib, u), R.encode_npu(xf))


def test_device_decode_matches_oracle(hostlib, R):
    y = np.empty(256, np.uint32)
    hostlib.chk_decode_bits(y.ctypes.data)
    d = R.decode_table()
    nan = np.isnan(d)
    assert np.array_equal(y[~nan], d[~nan].view(np.uint32))
    assert np.all(np.isnan(y.view(np.float32)[nan]))


def test_device_code_layout_known_answers(hostlib):
    """The kernels' decode of the published HiFloat8 layout's reference points (the same table
    test_oracle.py pins the oracle with)."""
    from test_oracle import HIF8_KNOWN
    y = np.empty(256, np.uint32)
    hostlib.chk_decode_bits(y.ctypes.data)
    d = y.view(np.float32)
    for c, v in HIF8_KNOWN.items():
        assert d[c] == v, (hex(c), d[c], v)
    assert np.isnan(d[0x80])
    vals = np.array([HIF8_KNOWN[c] for c in sorted(HIF8_KNOWN)], np.float32)
    assert np.array_equal(_enc(hostlib, vals.view(np.uint32)), np.array(sorted(HIF8_KNOWN), np.uint8))


def test_lds_encode_table(hostlib, R):
    buf = np.zeros(1 << 16, np.uint8)
    lo, hi = ctypes.c_uint32(), ctypes.c_uint32()
    n = hostlib.chk_table(buf.ctypes.data, ctypes.byref(lo), ctypes.byref(hi))
    tab = buf[:n]
    # kernel lookup: magnitude bits clamped to [lo, hi], entry = magnitude code
    u = np.arange(0, 0x7F81, dtype=np.uint32)      # every finite bf16 magnitude incl. Inf
    idx = np.clip(u, lo.value, hi.value) - lo.value
    xf = (u << 16).view(np.float32)
    assert np.array_equal(tab[idx], R.encode_npu(xf) & 0x7F)


def test_split_tail_plan_on_256_cus(pkg):
    """The split-tail plan (hif8_linear_split_workspace_bytes) as it is made for MI355X's 256 CUs
    (without a GPU the library assumes 256): only grids under 8 waves whose tail fills at most
    half the CUs split, into at most 8 ranges of at least 8 k-steps; 256 KB of fp32 per range."""
    L = pkg._lib.load()
    tile = 256 * 256 * 4
    assert L.hif8_linear_split_workspace_bytes(13824, 5120, 75600) == 56 * 4 * tile   # 1080 tiles: 4 ranges
    assert L.hif8_linear_split_workspace_bytes(4352, 4096, 4100) == 16 * 8 * tile     # 272 tiles: 8 ranges
    assert L.hif8_linear_split_workspace_bytes(4352, 4096, 1024) == 16 * 2 * tile     # 16 k-steps: 2 ranges
    assert L.hif8_linear_split_workspace_bytes(4352, 4096, 960) == 0                  # 15 k-steps: no split
    assert L.hif8_linear_split_workspace_bytes(75600, 5120, 13824) == 0               # 23 waves
    assert L.hif8_linear_split_workspace_bytes(4096, 4096, 75648) == 0                # whole waves
    assert L.hif8_linear_split_workspace_bytes(9216, 4096, 75648) == 64 * 4 * tile    # 576 tiles: tail of 64
    assert L.hif8_linear_split_workspace_bytes(12288, 5120, 75648) == 0               # tail of 192 > 128
