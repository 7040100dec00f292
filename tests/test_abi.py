"""CPU checks of the C ABI: the library loads, exports every function that
the headers under include/ declare, and rejects bad arguments with status codes
(no exception or abort crosses the ABI).  No kernel is launched here."""
import ctypes
import os
import re

import numpy as np
import pytest

import laguna_hip as lh
import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    names = set()
    inc = os.path.join(ROOT, "include")
    for f in sorted(os.listdir(inc)):
        if f.endswith(".h"):
            text = re.sub(r"/\*.*?\*/", "", open(os.path.join(inc, f)).read(), flags=re.S)
            names |= set(re.findall(r"\b(lg_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_header_and_binding_agree():
    declared = header_functions()
    assert declared, "no declarations found"
    assert set(declared) == set(lh.SIGNATURES), set(declared) ^ set(lh.SIGNATURES)


def test_library_exports_every_declared_symbol():
    L = lh.lib()
    for name in header_functions():
        assert hasattr(L, name), name


def test_version_and_device_count_without_gpu():
    assert b"gfx950" in lh.lib().lg_version()
    assert lh.device_count() >= 0


def _status(fn, *args):
    return getattr(lh.lib(), fn)(*args)


def test_null_pointers_are_einval():
    assert _status("lg_dispatch_proj_quant", None, None, None, 256, 4, lh.Q4_K, None) == lh.EINVAL
    assert b"null" in lh.lib().lg_last_error()
    assert _status("lg_dispatch_proj_quant_batch", None, lh.F32, None, None, 256, 4, 2, lh.Q4_K, None) == lh.EINVAL
    assert _status("lg_dispatch_activation", None, None, None, 4, None) == lh.EINVAL
    assert _status("lg_dequant_to_f32", None, 0, lh.Q8_0, 32, None, None) == lh.EINVAL


def test_bad_dtypes_are_einval():
    x = np.zeros(256, np.float32)
    c = np.zeros(4, np.float32)
    # host pointers are fine for argument validation: the call fails before any launch
    assert _status("lg_dispatch_proj_quant", x.ctypes.data, x.ctypes.data, c.ctypes.data, 256, 4, 13, None) == lh.EINVAL
    assert _status("lg_dispatch_proj_quant_batch", x.ctypes.data, lh.Q8_0, x.ctypes.data, c.ctypes.data, 256, 4, 1,
                   lh.Q4_K, None) == lh.EINVAL
    assert _status("lg_dispatch_proj_quant_batch", x.ctypes.data, lh.F32, x.ctypes.data, c.ctypes.data, 256, 4, 65,
                   lh.Q4_K, None) == lh.EINVAL


def test_zero_rows_is_a_no_op():
    # the reference dispatches ceil(0/256) = 0 workgroups
    assert _status("lg_dispatch_proj_quant", None, None, None, 256, 0, lh.Q4_K, None) == lh.OK
    assert _status("lg_dispatch_proj_quant_batch", None, lh.F32, None, None, 256, 0, 4, lh.Q4_K, None) == lh.OK


def test_buffer_calls_without_device_fail_cleanly():
    if lh.device_count() > 0:
        pytest.skip("host has a GPU")
    p = ctypes.c_void_p()
    st = lh.lib().lg_buf_alloc(ctypes.byref(p), 1024)
    assert st in (lh.ENOMEM, lh.EHIP, lh.ENODEV)
    assert lh.lib().lg_init(0) == lh.ENODEV


def test_synth_q8_0_quantizer_rule():
    x = synth.normal(1, 32 * 64, 0.02)
    raw = synth.quantize_q8_0(x).reshape(-1, 34)
    d = raw[:, 0:2].copy().view(np.float16)[:, 0].astype(np.float32)
    q = raw[:, 2:].view(np.int8).astype(np.float32)
    xb = x.reshape(-1, 32)
    amax = np.abs(xb).max(axis=1)
    assert np.array_equal(d, (amax / np.float32(127)).astype(np.float16).astype(np.float32))
    assert np.abs(q).max() <= 127 and np.abs(q).max(axis=1).min() == 127  # the max element maps to +-127
    # reconstruction error bounded by half a step of the unrounded scale
    assert np.all(np.abs(q * d[:, None] - xb) <= 0.5 * d[:, None] * 1.01 + 1e-3 * amax[:, None])


def test_synth_q4k_blocks():
    raw = synth.random_q4k(5, 1000).reshape(-1, 144)
    d = raw[:, 0:4].copy().view(np.float16).astype(np.float32)
    assert np.all((d >= 9.99e-5) & (d <= 4.01e-3))
    assert np.array_equal(synth.random_q4k(5, 1000), synth.random_q4k(5, 1000).copy())
    assert not np.array_equal(synth.random_q4k(5, 10), synth.random_q4k(6, 10))


def test_synth_normal_moments():
    z = synth.normal(0x5EED0002, 1 << 18).astype(np.float64)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01


def test_dflash_struct_layout_matches_header(tmp_path):
    """The ctypes mirrors of lg_dflash_hparams / lg_dflash_layer / lg_dflash_model
    have the C compiler's sizes and field offsets."""
    import shutil
    import subprocess

    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    checks = []
    for cname, cls in (("lg_dflash_hparams", lh._Hparams), ("lg_dflash_layer", lh._Layer),
                       ("lg_dflash_model", lh._Model)):
        checks.append((f"sizeof({cname})", ctypes.sizeof(cls)))
        for fname, _ in cls._fields_:
            checks.append((f"offsetof({cname}, {fname})", getattr(cls, fname).offset))
    src = tmp_path / "layout.c"
    src.write_text("#include <stddef.h>\n#include <stdio.h>\n#include \"laguna_hip.h\"\nint main(void) {\n"
                   + "".join(f'    printf("%zu\\n", (size_t){expr});\n' for expr, _ in checks) + "    return 0;\n}\n")
    exe = tmp_path / "layout"
    subprocess.run([cc, "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()]
    assert got == [v for _, v in checks], [(e, g, v) for (e, v), g in zip(checks, got) if g != v]


def test_dflash_rejects_bad_models_without_launching():
    import synth

    cfg = lh.DFlashConfig(n_embd=256, n_heads=4, n_kv=2, head_dim=64, rope_dim=32, n_ff=512, n_aux=2, n_layers=1)
    desc = lh._Model()
    desc.hp.n_embd, desc.hp.n_heads, desc.hp.n_kv_heads, desc.hp.head_dim = 256, 4, 2, 64
    desc.hp.rope_dim, desc.hp.n_ff, desc.hp.n_aux, desc.hp.n_layers = 32, 512, 2, 1
    layers = (lh._Layer * 1)()
    desc.layers = layers
    x = np.zeros(16, np.float32)
    p = x.ctypes.data
    # no layers' tensors, and a partial rotary dim: EINVAL before anything runs
    assert lh.lib().lg_dflash_forward_block(ctypes.byref(desc), p, p, 1, 0, p, None) == lh.EINVAL
    desc.hp.rope_dim = 64
    desc.enc_aux_norm = desc.fc = desc.enc_output_norm = p
    assert lh.lib().lg_dflash_forward_block(ctypes.byref(desc), p, p, 1, 0, p, None) == lh.EINVAL
    assert b"missing a tensor" in lh.lib().lg_last_error()
    assert lh.lib().lg_dflash_forward_block(ctypes.byref(desc), p, p, 33, 0, p, None) == lh.EINVAL
    assert lh.lib().lg_dflash_graph_create(ctypes.byref(desc), p, p, 1, 0, p, None, None) == lh.EINVAL
    assert lh.lib().lg_dispatch_qk_norm_rope(p, p, p, p, 2, 64, 32, 0, 1, 1e-6, None) == lh.EINVAL
    assert lh.lib().lg_dispatch_mha_attn(p, p, p, p, 3, 2, 64, 4, 0, 1, 1, None) == lh.EINVAL
    assert lh.lib().lg_dispatch_rmsnorm(None, p, p, 4, 1, 1e-5, None) == lh.EINVAL
    assert lh.lib().lg_dflash_graph_destroy(None) == lh.OK
    del cfg, synth
