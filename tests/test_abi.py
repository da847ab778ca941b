"""The C-ABI library: loads, exports what include/terra_swin.h declares, and
rejects bad arguments before any launch (all on the CPU, no kernel runs)."""
import ctypes
import os
import re

import pytest
import torch

import terra_amd._lib as L
from terra_amd import kernels

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "terra_swin.h")


def _declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(terra_\w+)\s*\(", text, flags=re.M)))


def test_header_and_binding_agree():
    assert _declared_functions() == sorted(L.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = L.load()
    for name in _declared_functions():
        assert hasattr(lib, name), name


def test_abi_version_and_struct_sizes():
    lib = L.load()
    assert lib.terra_abi_version() == L.ABI_VERSION
    text = open(HEADER).read()
    assert f"#define TERRA_SWIN_ABI_VERSION {L.ABI_VERSION}" in text
    # every field of the C structs is 4 bytes wide
    assert ctypes.sizeof(L.SwinGeom) == 4 * len(L.SwinGeom._fields_) == 60
    assert ctypes.sizeof(L.SwinAttnDesc) == 4 * len(L.SwinAttnDesc._fields_) == 92
    assert ctypes.sizeof(L.SwinBlockDesc) == 60 + 4 * (len(L.SwinBlockDesc._fields_) - 1) == 92
    assert ctypes.sizeof(L.SwinAttnBwdDesc) == 92 + 4 * 4 == 108
    assert ctypes.sizeof(L.SwinMlpDesc) == 4 * len(L.SwinMlpDesc._fields_) == 20


def _geom(**kw):
    g = L.SwinGeom()
    vals = dict(batch=1, height=16, width=16, channels=8, window=8)
    vals.update(kw)
    for k, v in vals.items():
        setattr(g, k, v)
    return g


FAKE = ctypes.c_void_p(1 << 20)  # never dereferenced: every case below fails validation


@pytest.mark.parametrize("kw,code,text", [
    (dict(height=15), -3, "not a multiple of window"),
    (dict(window=0), -3, "must be positive"),
    (dict(shift_h=16), -3, "shift"),
    (dict(pad_top=-1), -3, "non-negative"),
    (dict(win_row_begin=1, win_rows=2), -3, "window rows"),
    (dict(valid_begin=3, valid_end=2), -3, "valid window range"),
    (dict(valid_begin=0, valid_end=5), -3, "valid window range"),
])
def test_partition_rejects_bad_geometry(kw, code, text):
    lib = L.load()
    g = _geom(**kw)
    st = lib.terra_swin_partition(FAKE, FAKE, L.DTYPE_BF16, ctypes.byref(g), 0.0, None)
    assert st == code
    assert text in L.last_error()


def test_partition_rejects_null_and_dtype():
    lib = L.load()
    g = _geom()
    assert lib.terra_swin_partition(None, FAKE, L.DTYPE_BF16, ctypes.byref(g), 0.0, None) == -1
    assert lib.terra_swin_partition(FAKE, FAKE, 9, ctypes.byref(g), 0.0, None) == -2
    assert lib.terra_swin_partition(FAKE, FAKE, L.DTYPE_BF16, None, 0.0, None) == -1
    assert lib.terra_swin_reverse(FAKE, FAKE, FAKE, L.DTYPE_U8, ctypes.byref(g), None) == -2


def test_partition_rejects_misaligned_elements():
    lib = L.load()
    g = _geom()
    assert lib.terra_swin_partition(ctypes.c_void_p((1 << 20) + 1), FAKE, L.DTYPE_F32, ctypes.byref(g), 0.0,
                                    None) == -4


def _desc(**kw):
    d = L.SwinAttnDesc()
    vals = dict(num_windows=4, tokens=64, channels=64, heads=2, window_h=8, window_w=8, n_real=64,
                q_stride=64, k_stride=64, v_stride=64, o_stride=64, scale=0.17, mask_value=-100.0,
                pad_key_value=-10000.0, mask_mode=0)
    vals.update(kw)
    for k, v in vals.items():
        setattr(d, k, v)
    return d


@pytest.mark.parametrize("kw,code,text", [
    (dict(tokens=81, window_h=9, window_w=9, n_real=81), -5, "multiple of 128"),
    # windows of more than 64 tokens (the flash kernel): what it does not serve
    (dict(tokens=256, window_h=16, window_w=16, n_real=256, channels=96, heads=3, q_stride=96, k_stride=96,
          v_stride=96, o_stride=96), -5, "head dim 64 or 128"),
    (dict(tokens=256, window_h=16, window_w=8, n_real=256, channels=128, q_stride=128, k_stride=128, v_stride=128,
          o_stride=128), -3, "does not have 256 tokens"),
    (dict(tokens=256, window_h=16, window_w=16, n_real=200, channels=128, q_stride=128, k_stride=128,
          v_stride=128, o_stride=128), -5, "no padded keys"),
    (dict(tokens=256, window_h=16, window_w=16, n_real=256, channels=128, q_stride=128, k_stride=128,
          v_stride=128, o_stride=128, mask_mode=1), -5, "no mask"),
    (dict(tokens=256, window_h=16, window_w=16, n_real=256, channels=128, q_stride=128, k_stride=1 << 26,
          v_stride=128, o_stride=128), -3, "too large"),
    (dict(heads=3), -3, "not divisible"),
    (dict(channels=48, heads=3, q_stride=48, k_stride=48, v_stride=48, o_stride=48), -5, "head dim"),
    (dict(window_h=9), -5, "outside 1..8"),
    (dict(n_real=0), -3, "n_real"),
    (dict(q_stride=60), -3, ">= channels"),
    (dict(q_stride=68), -4, "multiples"),
    (dict(mask_mode=7), -3, "mask_mode"),
    (dict(mask_mode=2, mask_windows=4), -1, "explicit"),
    (dict(mask_mode=1, frame_h=16, frame_w=16, shift_h=4, shift_w=4, win_rows=2, win_cols=3), -3, "win_cols"),
    (dict(mask_mode=1, frame_h=16, frame_w=16, shift_h=8, shift_w=4, win_rows=2, win_cols=2), -3, "0 < shift"),
    (dict(mask_mode=1, frame_h=16, frame_w=24, shift_h=4, shift_w=4, win_rows=2, win_cols=3), -3, "multiple"),
])
def test_attention_rejects_bad_descriptors(kw, code, text):
    lib = L.load()
    d = _desc(**kw)
    st = lib.terra_swin_attn_fwd(FAKE, FAKE, FAKE, FAKE, L.DTYPE_BF16, ctypes.byref(d), None, None, None, None)
    assert st == code, L.last_error()
    assert text in L.last_error()


def test_attention_rejects_dtype_null_alignment():
    lib = L.load()
    d = _desc()
    assert lib.terra_swin_attn_fwd(FAKE, FAKE, FAKE, FAKE, L.DTYPE_F16, ctypes.byref(d), None, None, None,
                                   None) == -2
    assert lib.terra_swin_attn_fwd(None, FAKE, FAKE, FAKE, L.DTYPE_BF16, ctypes.byref(d), None, None, None,
                                   None) == -1
    bad = ctypes.c_void_p((1 << 20) + 8)
    assert lib.terra_swin_attn_fwd(bad, FAKE, FAKE, FAKE, L.DTYPE_BF16, ctypes.byref(d), None, None, None,
                                   None) == -4


def _bwd_desc(dout_stride=64, dq_stride=64, dk_stride=64, dv_stride=64, **kw):
    bd = L.SwinAttnBwdDesc()
    bd.fwd = _desc(**kw)
    bd.dout_stride, bd.dq_stride, bd.dk_stride, bd.dv_stride = dout_stride, dq_stride, dk_stride, dv_stride
    return bd


@pytest.mark.parametrize("kw,code,text", [
    (dict(tokens=81, window_h=9, window_w=9, n_real=81), -5, "multiple of 128"),
    # windows of more than 64 tokens (the flash backward): what it does not serve
    (dict(tokens=256, window_h=16, window_w=16, n_real=256, channels=128, q_stride=128, k_stride=128, v_stride=128,
          o_stride=128, dout_stride=128, dq_stride=128, dk_stride=128, dv_stride=128, scale=-0.1), -5,
     "positive finite scale"),
    (dict(tokens=256, window_h=16, window_w=16, n_real=256, channels=128, q_stride=128, k_stride=128, v_stride=128,
          o_stride=128, dout_stride=128, dq_stride=1 << 26, dk_stride=128, dv_stride=128), -3, "too large"),
    (dict(tokens=256, window_h=16, window_w=16, n_real=256, channels=128, q_stride=128, k_stride=128, v_stride=128,
          o_stride=128, dout_stride=128, dq_stride=128, dk_stride=128, dv_stride=128, mask_mode=1), -5, "no mask"),
    (dict(window_h=9), -5, "outside 1..8"),
    (dict(n_real=0), -3, "n_real"),
    (dict(heads=3), -3, "not divisible"),
    (dict(channels=48, heads=3, q_stride=48, k_stride=48, v_stride=48, o_stride=48, dout_stride=48,
          dq_stride=48, dk_stride=48, dv_stride=48), -5, "head dim"),
    (dict(dq_stride=60), -3, ">= channels"),
    (dict(dv_stride=68), -4, "multiples"),
    (dict(mask_mode=7), -3, "mask_mode"),
    (dict(mask_mode=2, mask_windows=4), -1, "explicit"),
    (dict(mask_mode=1, frame_h=16, frame_w=16, shift_h=4, shift_w=4, win_rows=2, win_cols=3), -3, "win_cols"),
])
def test_attention_backward_rejects_bad_descriptors(kw, code, text):
    lib = L.load()
    bd = _bwd_desc(**kw)
    st = lib.terra_swin_attn_bwd(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, L.DTYPE_BF16, ctypes.byref(bd), None, None,
                                 None, None, None)
    assert st == code, L.last_error()
    assert text in L.last_error()


def test_attention_backward_rejects_dtype_null_alignment_table():
    lib = L.load()
    bd = _bwd_desc()
    call = lambda *a: lib.terra_swin_attn_bwd(*a, ctypes.byref(bd), None, None, None, None, None)  # noqa: E731
    assert call(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, L.DTYPE_F16) == -2
    assert call(FAKE, FAKE, FAKE, FAKE, None, FAKE, FAKE, L.DTYPE_BF16) == -1
    bad = ctypes.c_void_p((1 << 20) + 8)
    assert call(FAKE, FAKE, FAKE, FAKE, FAKE, bad, FAKE, L.DTYPE_BF16) == -4
    # a bias-table gradient needs the bias table
    st = lib.terra_swin_attn_bwd(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, L.DTYPE_BF16, ctypes.byref(bd), None,
                                 FAKE, None, None, None)
    assert st == -3 and "dbias_table" in L.last_error()


def test_python_wrapper_raises_instead_of_falling_back():
    x = torch.zeros(1, 16, 16, 8)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        kernels.swin_partition(x, kernels.WindowGeometry(1, 16, 16, 8, 8))
    q = torch.zeros(2, 64, 64)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        kernels.window_attention(q, q, q, 2, (8, 8), 0.1)
    qb = q.to(torch.bfloat16)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        kernels.window_attention_backward(qb, qb, qb, qb, 2, (8, 8), 0.1)


def test_check_maps_status_to_exceptions():
    with pytest.raises(ValueError, match="TERRA_ERR_SHAPE"):
        L.check(-3, "x")
    with pytest.raises(L.TerraError):
        L.check(-6, "x")
    L.check(0, "x")


def test_partition_ln_rejects_bad_arguments():
    lib = L.load()
    g = _geom(channels=8)  # bf16: 16-byte rows
    assert lib.terra_swin_partition_ln(FAKE, FAKE, L.DTYPE_U8, ctypes.byref(g), None, None, 1e-5, 0.0, None) == -2
    assert lib.terra_swin_partition_ln(None, FAKE, L.DTYPE_BF16, ctypes.byref(g), None, None, 1e-5, 0.0, None) == -1
    g6 = _geom(channels=6)  # 12-byte rows
    assert lib.terra_swin_partition_ln(FAKE, FAKE, L.DTYPE_BF16, ctypes.byref(g6), None, None, 1e-5, 0.0, None) == -4
    big = _geom(channels=1032)  # more than 1024 channels
    assert lib.terra_swin_partition_ln(FAKE, FAKE, L.DTYPE_BF16, ctypes.byref(big), None, None, 1e-5, 0.0, None) == -5
    assert "1024 channels" in L.last_error()
    assert lib.terra_swin_partition_ln(FAKE, FAKE, L.DTYPE_BF16, ctypes.byref(g), None, None, -1.0, 0.0, None) == -3


def test_partition_ln_mixed_rejects_bad_arguments():
    lib = L.load()
    g = _geom(channels=8)
    mixed = lib.terra_swin_partition_ln_mixed
    # only fp32 x with bf16 windows mixes
    assert mixed(FAKE, L.DTYPE_BF16, FAKE, L.DTYPE_F32, ctypes.byref(g), None, None, 1e-5, 0.0, None) == -2
    assert "mixed" in L.last_error()
    assert mixed(FAKE, L.DTYPE_F32, FAKE, L.DTYPE_F16, ctypes.byref(g), None, None, 1e-5, 0.0, None) == -2
    assert mixed(None, L.DTYPE_F32, FAKE, L.DTYPE_BF16, ctypes.byref(g), None, None, 1e-5, 0.0, None) == -1
    assert mixed(FAKE, L.DTYPE_F32, FAKE, L.DTYPE_BF16, ctypes.byref(g), None, None, -1.0, 0.0, None) == -3
    bwd = lib.terra_swin_partition_ln_bwd_mixed
    assert bwd(FAKE, L.DTYPE_F32, FAKE, None, FAKE, L.DTYPE_BF16, ctypes.byref(g), None, 1e-5, None, None,
               None) == -2
    assert bwd(None, L.DTYPE_BF16, FAKE, None, FAKE, L.DTYPE_F32, ctypes.byref(g), None, 1e-5, None, None,
               None) == -1
    assert bwd(FAKE, L.DTYPE_BF16, FAKE, None, FAKE, L.DTYPE_F32, ctypes.byref(g), None, -1.0, None, None,
               None) == -3


def test_mixed_copies_reject_bad_arguments():
    lib = L.load()
    g = _geom(channels=8)
    part = lib.terra_swin_partition_mixed
    # only fp32 x into bf16 windows
    assert part(FAKE, L.DTYPE_BF16, FAKE, L.DTYPE_F32, ctypes.byref(g), 0.0, None, None) == -2
    assert "mixed partition" in L.last_error()
    assert part(FAKE, L.DTYPE_F32, FAKE, L.DTYPE_F32, ctypes.byref(g), 0.0, None, None) == -2
    assert part(None, L.DTYPE_F32, FAKE, L.DTYPE_BF16, ctypes.byref(g), 0.0, None, None) == -1
    assert part(FAKE, L.DTYPE_F32, FAKE, L.DTYPE_BF16, None, 0.0, None, None) == -1
    assert part(FAKE, L.DTYPE_F32, FAKE, L.DTYPE_BF16, ctypes.byref(_geom(channels=6)), 0.0, None, None) == -4
    assert part(FAKE, L.DTYPE_F32, ctypes.c_void_p((1 << 20) + 4), L.DTYPE_BF16, ctypes.byref(g), 0.0, None,
                None) == -4
    assert part(FAKE, L.DTYPE_F32, FAKE, L.DTYPE_BF16, ctypes.byref(g), 0.0, ctypes.c_void_p((1 << 20) + 2),
                None) == -4
    assert part(FAKE, L.DTYPE_F32, FAKE, L.DTYPE_BF16, ctypes.byref(_geom(channels=1028)), 0.0, None, None) == -5
    assert part(FAKE, L.DTYPE_F32, FAKE, L.DTYPE_BF16, ctypes.byref(_geom(height=15)), 0.0, None, None) == -3
    rev = lib.terra_swin_reverse_mixed
    assert rev(FAKE, L.DTYPE_F32, FAKE, None, L.DTYPE_BF16, ctypes.byref(g), None) == -2
    assert "mixed reverse" in L.last_error()
    assert rev(FAKE, L.DTYPE_BF16, FAKE, None, L.DTYPE_F16, ctypes.byref(g), None) == -2
    assert rev(None, L.DTYPE_BF16, FAKE, None, L.DTYPE_F32, ctypes.byref(g), None) == -1
    assert rev(FAKE, L.DTYPE_BF16, None, None, L.DTYPE_F32, ctypes.byref(g), None) == -1
    assert rev(ctypes.c_void_p((1 << 20) + 4), L.DTYPE_BF16, FAKE, None, L.DTYPE_F32, ctypes.byref(g), None) == -4
    assert rev(FAKE, L.DTYPE_BF16, FAKE, ctypes.c_void_p((1 << 20) + 8), L.DTYPE_F32, ctypes.byref(g), None) == -4
    assert rev(FAKE, L.DTYPE_BF16, FAKE, None, L.DTYPE_F32, ctypes.byref(_geom(window=0)), None) == -3


def test_gelu_bwd_rejects_bad_arguments():
    gelu = L.load().terra_swin_gelu_bwd
    other = ctypes.c_void_p(1 << 30)
    dh = ctypes.c_void_p(1 << 31)
    assert gelu(None, other, dh, L.DTYPE_BF16, 4, 64, None, None) == -1
    assert gelu(FAKE, other, None, L.DTYPE_BF16, 4, 64, None, None) == -1
    assert gelu(FAKE, other, dh, L.DTYPE_F16, 4, 64, None, None) == -2
    assert gelu(FAKE, other, dh, L.DTYPE_BF16, -1, 64, None, None) == -3
    assert gelu(FAKE, other, dh, L.DTYPE_BF16, 4, 0, None, None) == -3
    assert gelu(FAKE, other, dh, L.DTYPE_BF16, 4, 12, None, None) == -4     # 24-byte rows
    assert "16-byte" in L.last_error()
    assert gelu(FAKE, other, dh, L.DTYPE_BF16, 4, 4104, None, None) == -5   # rows over 8192 bytes
    assert gelu(FAKE, other, dh, L.DTYPE_F32, 4, 2056, None, None) == -5
    assert gelu(ctypes.c_void_p((1 << 20) + 8), other, dh, L.DTYPE_BF16, 4, 64, None, None) == -4
    assert gelu(FAKE, other, dh, L.DTYPE_BF16, 4, 64, ctypes.c_void_p((1 << 20) + 2), None) == -4
    assert gelu(FAKE, other, FAKE, L.DTYPE_BF16, 4, 64, None, None) == -3   # dh is dout
    assert "overlap" in L.last_error()
    assert gelu(FAKE, other, ctypes.c_void_p((1 << 30) + 64), L.DTYPE_BF16, 4, 64, None, None) == -3
    assert gelu(FAKE, other, dh, L.DTYPE_BF16, 0, 64, None, None) == 0      # no rows: nothing launched


def _block_desc(geom_kw=None, **kw):
    d = L.SwinBlockDesc()
    gk = dict(channels=192, window=8)
    gk.update(geom_kw or {})
    d.geom = _geom(**gk)
    vals = dict(heads=6, scale=32 ** -0.5, ln_eps=1e-5, mask_value=-100.0, layernorm=1, shift_mask=0,
                land_windows=0)
    vals.update(kw)
    for k, v in vals.items():
        setattr(d, k, v)
    return d


def _block_call(d, dtype=L.DTYPE_BF16, x=FAKE, land=None):
    return L.load().terra_swin_block_fwd(x, FAKE, dtype, ctypes.byref(d) if d is not None else None, None, None,
                                         FAKE, None, FAKE, None, None, land, None)


@pytest.mark.parametrize("geom_kw,kw,dtype,code,text", [
    ({}, {}, L.DTYPE_F32, -5, "bf16 only"),
    ({}, {}, 9, -2, "unknown dtype"),
    ({"window": 4}, {}, L.DTYPE_BF16, -5, "8x8 windows"),
    ({"window": 7, "height": 14, "width": 14}, {}, L.DTYPE_BF16, -5, "7x7 windows with 4 heads"),
    ({"channels": 128}, {"heads": 4}, L.DTYPE_BF16, -5, "6 or 12 heads"),
    ({"channels": 384}, {"heads": 6}, L.DTYPE_BF16, -5, "head dim 32"),
    ({"height": 12}, {}, L.DTYPE_BF16, -3, "not a multiple of window"),
    ({"valid_begin": 0, "valid_end": 9}, {}, L.DTYPE_BF16, -3, "valid window range"),
    ({}, {"ln_eps": -1.0}, L.DTYPE_BF16, -3, "ln_eps"),
])
def test_block_rejects_bad_descriptors(geom_kw, kw, dtype, code, text):
    st = _block_call(_block_desc(geom_kw, **kw), dtype)
    assert st == code, L.last_error()
    assert text in L.last_error()


def test_block_rejects_null_alignment_overlap_land():
    d = _block_desc()
    assert _block_call(None) == -1
    assert _block_call(d, x=None) == -1
    assert _block_call(d, x=ctypes.c_void_p((1 << 20) + 8)) == -4
    assert _block_call(d, land=FAKE) == -3  # land bits without a period
    assert "land_windows" in L.last_error()
    g = _geom(channels=192, window=8)
    n_we = (g.height // 8) * (g.width // 8)
    for bad in (n_we - 1, n_we + 1, 3 * n_we if g.batch % 3 else 5 * n_we):  # not whole images dividing the batch
        assert _block_call(_block_desc(land_windows=bad), land=FAKE) == -3
        assert "land_windows" in L.last_error()
    lib = L.load()
    y = ctypes.c_void_p((1 << 20) + 4096)  # overlaps x without being x
    assert lib.terra_swin_block_fwd(FAKE, y, L.DTYPE_BF16, ctypes.byref(d), None, None, FAKE, None, FAKE, None,
                                    None, None, None) == -3
    assert "overlaps" in L.last_error()


def test_block_wrapper_raises_on_cpu_tensors():
    x = torch.zeros(1, 16, 16, 192, dtype=torch.bfloat16)
    w = torch.zeros(576, 192, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        kernels.swin_block(x, kernels.WindowGeometry(1, 16, 16, 192, 8), 6, 0.17, w, None, w[:192], None)


def test_pack_linear_rejects_bad_arguments():
    lib = L.load()
    assert lib.terra_swin_pack_linear(None, FAKE, L.DTYPE_BF16, 16, 32, None) == -1
    assert lib.terra_swin_pack_linear(FAKE, FAKE, L.DTYPE_F32, 16, 32, None) == -5
    assert lib.terra_swin_pack_linear(FAKE, FAKE, L.DTYPE_BF16, 24, 32, None) == -3
    assert lib.terra_swin_pack_linear(FAKE, FAKE, L.DTYPE_BF16, 16, 48, None) == -3
    assert lib.terra_swin_pack_linear(ctypes.c_void_p((1 << 20) + 2), ctypes.c_void_p(1 << 24), L.DTYPE_BF16,
                                      16, 32, None) == -4
    assert lib.terra_swin_pack_linear(FAKE, FAKE, L.DTYPE_BF16, 16, 32, None) == -3  # overlap


def _mlp_desc(**kw):
    d = L.SwinMlpDesc()
    vals = dict(tokens=100, channels=192, hidden=768, layernorm=1, ln_eps=1e-5)
    vals.update(kw)
    for k, v in vals.items():
        setattr(d, k, v)
    return d


def _mlp_call(d, dtype=L.DTYPE_BF16, x=FAKE, y=ctypes.c_void_p(1 << 24), w1=FAKE, b1=None):
    return L.load().terra_swin_mlp_fwd(x, y, dtype, ctypes.byref(d) if d is not None else None, None, None,
                                       w1, b1, FAKE, None, None)


@pytest.mark.parametrize("kw,dtype,code,text", [
    ({}, L.DTYPE_F32, -5, "bf16 activations"),
    ({}, 9, -2, "unknown dtype"),
    ({"channels": 256, "hidden": 1024}, L.DTYPE_BF16, -5, "not in {128, 192, 384, 768}"),
    ({"hidden": 576}, L.DTYPE_BF16, -5, "4 * channels"),
    ({"tokens": 0}, L.DTYPE_BF16, -3, "tokens must be positive"),
    ({"ln_eps": -1.0}, L.DTYPE_BF16, -3, "ln_eps"),
    ({"tokens": 1 << 30}, L.DTYPE_BF16, -3, "under 4 GiB"),
])
def test_mlp_rejects_bad_descriptors(kw, dtype, code, text):
    st = _mlp_call(_mlp_desc(**kw), dtype)
    assert st == code, L.last_error()
    assert text in L.last_error()


def test_mlp_rejects_null_alignment_overlap():
    d = _mlp_desc()
    assert _mlp_call(None) == -1
    assert _mlp_call(d, x=None) == -1
    assert _mlp_call(d, w1=None) == -1
    assert _mlp_call(d, x=ctypes.c_void_p((1 << 20) + 8)) == -4
    assert _mlp_call(d, b1=ctypes.c_void_p((1 << 20) + 4)) == -4
    assert _mlp_call(d, y=ctypes.c_void_p((1 << 20) + 4096)) == -3  # overlaps x without being x
    assert "overlaps" in L.last_error()


def test_mlp_wrapper_raises_on_cpu_tensors():
    x = torch.zeros(64, 192, dtype=torch.bfloat16)
    w = torch.zeros(768 * 192, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        kernels.swin_mlp(x, w, None, w, None)
    from terra_amd.mlp import SequentialMlp
    with pytest.raises(RuntimeError, match="device tensors only"):
        SequentialMlp(192, 768)(x.float())


def _lin_call(x=FAKE, y=ctypes.c_void_p(1 << 30), dtype=L.DTYPE_BF16, rows=512, k=1024, n=1024, xs=None, ys=None,
              w=FAKE, b=None, epi=0):
    return L.load().terra_swin_linear(x, y, dtype, rows, k, n, k if xs is None else xs, n if ys is None else ys, w,
                                      b, epi, None)


def test_linear_rejects_bad_arguments():
    assert _lin_call(x=None) == -1
    assert _lin_call(w=None) == -1
    assert _lin_call(dtype=L.DTYPE_F32) == -5 and "bf16 only" in L.last_error()
    assert _lin_call(dtype=9) == -2
    assert _lin_call(n=192) == -3 and "multiple" in L.last_error()
    assert _lin_call(k=48) == -3
    assert _lin_call(rows=-1) == -3
    assert _lin_call(xs=1000) == -3 and "row strides" in L.last_error()
    assert _lin_call(ys=1022) == -3
    assert _lin_call(x=ctypes.c_void_p((1 << 20) + 8)) == -4
    assert _lin_call(b=ctypes.c_void_p((1 << 20) + 4)) == -4
    assert _lin_call(epi=7) == -3 and "epilogue" in L.last_error()
    assert _lin_call(y=ctypes.c_void_p((1 << 20) + 4096)) == -3 and "overlaps" in L.last_error()
    assert _lin_call(rows=0) == 0  # nothing to do, nothing launched


def _lin_res_call(x=FAKE, r=ctypes.c_void_p(1 << 31), y=ctypes.c_void_p(1 << 31), rows=512, k=1024, n=1024, geom=None):
    return L.load().terra_swin_linear_residual(x, r, y, L.DTYPE_BF16, rows, k, n, FAKE, None,
                                               None if geom is None else ctypes.byref(geom), None)


def test_linear_residual_rejects_bad_arguments():
    assert _lin_res_call(r=None) == -1
    assert _lin_res_call(r=ctypes.c_void_p((1 << 31) + 4)) == -4
    assert _lin_res_call(y=ctypes.c_void_p((1 << 31) + 4096)) == -3 and "overlaps residual" in L.last_error()
    full = kernels.WindowGeometry(1, 16, 24, 1024, 8, 4, 4).to_c()
    slab = kernels.WindowGeometry(1, 16, 24, 1024, 8, 4, 4, (0, 0, 0, 0), 0, 1).to_c()
    assert _lin_res_call(rows=3 * 64, geom=slab) == -5 and "every window of the frame" in L.last_error()
    w7 = kernels.WindowGeometry(1, 14, 21, 1024, 7).to_c()
    assert _lin_res_call(rows=6 * 49, geom=w7) == -5 and "8x8 windows" in L.last_error()
    assert _lin_res_call(rows=5 * 64, geom=full) == -3 and "window tokens" in L.last_error()
    other_c = kernels.WindowGeometry(1, 16, 24, 768, 8).to_c()
    assert _lin_res_call(rows=6 * 64, geom=other_c) == -3 and "out_features" in L.last_error()
