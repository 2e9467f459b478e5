"""C-ABI checks that need no GPU: the library loads, exports every entry point
include/dgattn.h declares, reports its ABI version, and rejects bad arguments
with a status code and a message before touching the device."""

import ctypes
import re

import pytest

from conftest import REPO


def _declared_symbols():
    text = (REPO / "include" / "dgattn.h").read_text()
    return sorted(set(re.findall(r"DG_API\s+[\w\s\*]+?\b(dg_\w+)\s*\(", text)))


def test_header_declares_the_entry_points():
    syms = _declared_symbols()
    assert {"dg_abi_version", "dg_last_error", "dg_rope_qknorm_append", "dg_attention",
            "dg_attention_grouped", "dg_attention_workspace_size", "dg_rms_norm",
            "dg_copy4d", "dg_decode_step", "dg_decode_step_workspace_size"} <= set(syms)


def test_library_exports_every_declared_symbol():
    from diff_gpt import _native

    lib = _native.lib()
    for name in _declared_symbols():
        assert hasattr(lib, name), f"libdgattn.so does not export {name}"
    assert lib.dg_abi_version() == _native.ABI_VERSION


def _s3(b=0, t=0, h=0):
    from diff_gpt._native import Stride3

    return ctypes.pointer(Stride3(b, t, h))


def test_argument_errors_return_status_and_message():
    from diff_gpt import _native

    lib = _native.lib()
    nul = ctypes.c_void_p(0)
    fake = ctypes.c_void_p(0x1000)
    # odd head_dim
    rc = lib.dg_rope_qknorm_append(1, 1, 1, 5, 0, fake, _s3(), fake, _s3(), nul, None, nul, None,
                                   nul, None, nul, None, fake, _s3(), 0, 1, nul)
    assert rc == -1 and b"even" in lib.dg_last_error()
    # unsupported dtype
    rc = lib.dg_attention(1, 1, 1, 1, 16, 7, fake, _s3(), fake, _s3(), fake, _s3(), fake, _s3(),
                          1.0, nul, 0, nul)
    assert rc == -2 and b"dtype" in lib.dg_last_error()
    # Tk < Tq
    rc = lib.dg_attention(1, 1, 4, 2, 16, 0, fake, _s3(), fake, _s3(), fake, _s3(), fake, _s3(),
                          1.0, nul, 0, nul)
    assert rc == -1 and b"Tk" in lib.dg_last_error()
    # rms_norm row too long
    rc = lib.dg_rms_norm(1, 10000, 0, fake, 10000, fake, 10000, nul)
    assert rc == -2
    # grouped attention: group < 1, a prefix longer than the keys, own pages
    # without prefix pages, prefix pages with another position stride
    rc = lib.dg_attention_grouped(1, 1, 1, 8, 16, 0, fake, _s3(), fake, _s3(), fake, _s3(), fake,
                                  _s3(), 1.0, _prefix(4, 0), nul, 0, nul)
    assert rc == -1 and b"group" in lib.dg_last_error()
    rc = lib.dg_attention_grouped(1, 1, 1, 8, 16, 0, fake, _s3(), fake, _s3(), fake, _s3(), fake,
                                  _s3(), 1.0, _prefix(9, 2), nul, 0, nul)
    assert rc == -1 and b"prefix len" in lib.dg_last_error()
    rc = lib.dg_attention_grouped(1, 1, 1, 8, 16, 0, fake, _s3(), fake, _s3(), fake, _s3(), fake,
                                  _s3(), 1.0, _prefix(4, 2, own_start=4), nul, 0, nul)
    assert rc == -1 and b"own_start" in lib.dg_last_error()
    rc = lib.dg_attention_grouped(1, 1, 1, 8, 16, 0, fake, _s3(0, 16, 0), fake, _s3(0, 16, 0), fake, _s3(), fake,
                                  _s3(), 1.0, _prefix(4, 2, pages=True, t=32), nul, 0, nul)
    assert rc == -1 and b"position stride" in lib.dg_last_error()
    # empty work is a no-op success
    assert lib.dg_attention(0, 1, 1, 1, 16, 0, nul, _s3(), nul, _s3(), nul, _s3(), nul, _s3(),
                            1.0, nul, 0, nul) == 0


def _prefix(length, group, own_start=0, pages=False, t=0):
    from diff_gpt._native import DgPrefix, Stride3

    p = DgPrefix()
    p.len, p.group, p.own_start = length, group, own_start
    if pages:
        p.k = p.v = 0x2000
        p.k_st = p.v_st = Stride3(0, t, 0)
    return ctypes.pointer(p)


def _decode_step(lib, pos, max_pos=8, prefix_len=0, group=1, dtype=0, D=16, B=1):
    fake = ctypes.c_void_p(0x1000)
    nul = ctypes.c_void_p(0)
    return lib.dg_decode_step(B, 1, D, dtype, fake, _s3(), fake, _s3(), fake, _s3(), fake, _s3(), fake, _s3(),
                              fake, 0, 0, pos, nul, max_pos, fake, _s3(), 0.25, _prefix(prefix_len, group), 1,
                              nul, 0, nul)


def test_decode_step_argument_errors():
    """dg_decode_step rejects a host position outside the cache or inside the
    shared prefix, bad dtypes and odd head dims before any launch."""
    from diff_gpt import _native

    lib = _native.lib()
    assert _decode_step(lib, pos=8) == -1 and b"position" in lib.dg_last_error()
    assert _decode_step(lib, pos=-1) == -1 and b"position" in lib.dg_last_error()
    assert _decode_step(lib, pos=3, prefix_len=5, group=4) == -1 and b"prefix" in lib.dg_last_error()
    assert _decode_step(lib, pos=3, prefix_len=9, group=4) == -1 and b"prefix len" in lib.dg_last_error()
    assert _decode_step(lib, pos=3, dtype=7) == -2 and b"dtype" in lib.dg_last_error()
    assert _decode_step(lib, pos=3, D=15) == -1 and b"even" in lib.dg_last_error()
    assert _decode_step(lib, pos=3, max_pos=0) == -1 and b"max_pos" in lib.dg_last_error()
    assert _decode_step(lib, pos=3, B=0) == 0  # empty work


def test_workspace_sizes():
    from diff_gpt import _native

    lib = _native.lib()
    # many rows: no split, no workspace
    assert lib.dg_attention_workspace_size(6400, 4, 1, 144, 16, 0) == 0
    # cfg4 decode: 8 key splits per (row, head), merged inside the workgroup
    assert lib.dg_attention_workspace_size(64, 8, 1, 3680, 128, 1) == 0
    # very few long rows: more than 16 splits, partials of (D + 2) fp32 per unit
    ws = lib.dg_attention_workspace_size(1, 8, 1, 8192, 128, 1)
    assert ws == 8 * 64 * 130 * 4
    # prefill never splits
    assert lib.dg_attention_workspace_size(1, 1, 512, 512, 64, 1) == 0


def test_float64_declined_where_no_float64_form():
    """dg_prefill_rope, dg_lm_head and dg_block_out have no float64 kernels:
    they return DG_EUNSUPPORTED (the model then makes the separate calls)
    before touching the device; an unknown dtype code is refused everywhere."""
    from diff_gpt import _native

    lib = _native.lib()
    nul = ctypes.c_void_p(0)
    fake = ctypes.c_void_p(0x1000)
    st = _s3(64, 64, 64)
    F64 = _native.DG_F64
    assert lib.dg_prefill_rope(1, 1, 32, 32, 64, F64, fake, st, fake, st, F64, 1, fake, st, fake, st,
                               fake, st, 0.125, nul) == -2
    assert lib.dg_lm_head(4, 64, 256, F64, fake, 64, fake, 64, 15.0, fake, 256, nul, nul) == -2
    ptrs = (ctypes.c_void_p * 1)(0x1000)
    lds = (ctypes.c_int64 * 1)(64)
    assert lib.dg_block_out(16, 64, F64, fake, 64, fake, 64, fake, 64, nul, 0, 1, ptrs, lds, fake, fake, 64,
                            fake, 128, 1.702, 7.0, fake, 64, nul) == -2
    assert b"dtype" in lib.dg_last_error()
    assert lib.dg_block_out_norm(16, 64, 0, fake, 64, fake, 64, fake, 64, nul, 0, 1, ptrs, lds, fake, fake, 64,
                                 fake, 128, 1.702, 7.0, fake, 64, nul, 64, nul) == -1
    assert b"NULL" in lib.dg_last_error()
    assert lib.dg_block_out_norm(16, 96, 0, fake, 96, fake, 96, fake, 96, nul, 0, 1, ptrs, lds, fake, fake, 96,
                                 fake, 192, 1.702, 7.0, fake, 96, fake, 96, nul) == -2
    assert lib.dg_draw_argmax(4, 256, 5, fake, 256, fake, 256, fake, nul) == -2
    assert lib.dg_draw_argmax(4, 256, 0, fake, 128, fake, 256, fake, nul) == -1
    assert lib.dg_draw_argmax(0, 256, 0, nul, 256, nul, 256, nul, nul) == 0
    assert lib.dg_attention_workspace_size(1, 1, 1, 4096, 64, F64) == 0
    assert lib.dg_rms_norm(4, 64, 4, fake, 64, fake, 64, nul) == -2
    assert lib.dg_embed_norm(4, 64, F64, fake, 8, fake, 64, fake, 64, nul, 64, nul) == -2
    assert b"dtype" in lib.dg_last_error()
    # embed_norm: empty table, row too long, stride below C; no rows is a no-op
    assert lib.dg_embed_norm(4, 64, 0, fake, 0, fake, 64, fake, 64, nul, 64, nul) == -1
    assert lib.dg_embed_norm(4, 10000, 0, fake, 8, fake, 10000, fake, 10000, nul, 10000, nul) == -2
    assert lib.dg_embed_norm(4, 64, 0, fake, 8, fake, 32, fake, 64, nul, 64, nul) == -1
    assert lib.dg_embed_norm(0, 64, 0, nul, 8, nul, 64, nul, 64, nul, 64, nul) == 0


def test_block_kernel_argument_errors():
    """The decode-step neighbour kernels reject bad sizes before any launch."""
    from diff_gpt import _native

    lib = _native.lib()
    nul = ctypes.c_void_p(0)
    fake = ctypes.c_void_p(0x1000)
    ptrs = (ctypes.c_void_p * 33)(*([0x1000] * 33))
    lds = (ctypes.c_int64 * 33)(*([64] * 33))
    # no sources / too many sources
    assert lib.dg_attn_res_norm(4, 64, 0, 0, ptrs, lds, fake, fake, 64, nul) == -1
    assert b"sources" in lib.dg_last_error()
    assert lib.dg_attn_res_norm(4, 64, 0, 33, ptrs, lds, fake, fake, 64, nul) == -1
    # row longer than supported, unsupported dtype
    assert lib.dg_attn_res_norm(4, 4096, 0, 2, ptrs, lds, fake, fake, 4096, nul) == -2
    assert lib.dg_attn_res_norm(4, 64, 9, 2, ptrs, lds, fake, fake, 64, nul) == -2
    # a source row stride shorter than C
    short = (ctypes.c_int64 * 2)(64, 32)
    assert lib.dg_attn_res_norm(4, 64, 0, 2, ptrs, short, fake, fake, 64, nul) == -1
    assert b"stride" in lib.dg_last_error()
    # swiglu input rows hold 2N elements
    assert lib.dg_swiglu(4, 64, 0, fake, 64, fake, 64, 1.702, 7.0, nul) == -1
    # soft cap must be positive
    assert lib.dg_softcap(4, 64, 0, fake, 64, fake, 64, 0.0, nul) == -1
    assert b"cap" in lib.dg_last_error()
    # gate with a short row stride
    assert lib.dg_gate(4, 64, 0, fake, 64, fake, 8, fake, 64, nul) == -1
    # zero rows is a no-op
    assert lib.dg_gate(0, 64, 0, nul, 64, nul, 64, nul, 64, nul) == 0
