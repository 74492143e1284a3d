"""The C-ABI library loads and exports every entry point include/tinybatch_amd.h declares.

No kernel is launched: the argument checks below return before any HIP call,
so these run on a machine without a GPU.
"""
import ctypes
import os
import re
import subprocess

import pytest

from tinybatch_amd import _lib
from tinybatch_amd.build import LIB_PATH

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "tinybatch_amd.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^(?:const char\*|int32_t|size_t)\s+(tb_\w+)\(", text, re.M)))


def test_library_built():
    assert os.path.exists(LIB_PATH), "run python -m tinybatch_amd.build"


def test_every_declared_symbol_is_exported():
    names = _declared()
    assert len(names) >= 9
    out = subprocess.run(["nm", "-D", "--defined-only", LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if l.strip()}
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    # and the ctypes binding covers exactly the header
    assert sorted(_lib.SIGNATURES) == names


def test_status_strings():
    L = _lib.lib()
    assert L.tb_status_string(0) == b"ok"
    assert b"invalid" in L.tb_status_string(-1)
    assert b"unsupported" in L.tb_status_string(-2)


def test_append_rejects_bad_arguments_without_launching():
    L = _lib.lib()
    fake = ctypes.c_void_p(4096)
    # unknown dtype
    assert L.tb_kv_append(fake, 128, fake, 128, fake, 16, fake, 4, 2, 64, 16, 7, None) == _lib.TB_ERR_INVALID_ARG
    # block size not a power of two
    assert L.tb_kv_append(fake, 128, fake, 128, fake, 16, fake, 4, 2, 64, 12, 1, None) == _lib.TB_ERR_INVALID_ARG
    # head_dim whose rows are not whole 16-byte vectors
    assert L.tb_kv_append(fake, 120, fake, 120, fake, 16, fake, 4, 2, 60, 16, 1, None) == _lib.TB_ERR_UNSUPPORTED
    # zero tokens is a no-op
    assert L.tb_kv_append(None, 128, None, 128, fake, 16, None, 0, 2, 64, 16, 1, None) == _lib.TB_OK
    # the RoPE append: tables required, each half a whole number of 16-byte chunks
    ap = L.tb_kv_append_rope
    assert ap(fake, 128, fake, 128, fake, 16, fake, fake, None, fake, 64, 4, 2, 64, 16, 1, None) == _lib.TB_ERR_INVALID_ARG
    assert ap(fake, 128, fake, 128, fake, 16, fake, fake, fake, fake, 0, 4, 2, 64, 16, 1, None) == _lib.TB_ERR_INVALID_ARG
    assert ap(fake, 128, fake, 128, fake, 16, fake, fake, fake, fake, 64, 4, 2, 8, 16, 1, None) == _lib.TB_ERR_UNSUPPORTED
    assert ap(None, 128, None, 128, fake, 16, None, None, None, None, 0, 0, 2, 64, 16, 1, None) == _lib.TB_OK


def test_attention_rejects_bad_arguments_without_launching():
    L = _lib.lib()
    f = ctypes.c_void_p(4096)

    def call(**kw):
        a = dict(q=f, qs=896, pool=f, nb=64, out=f, os=896, bt=f, mnb=4, work=f, nw=2, tiles=None, nt=0,
                 rpo=f, nr=2, split=None, ns=0, mpr=1, pt=256, tp=2, hq=14, hkv=2, d=64, bs=16, scale=0.125,
                 dt=1, kn=None, ks=0, vn=None, vs=0, ws=None, wsb=0, rc=None, rs=None, rmax=0)
        a.update(kw)
        return L.tb_paged_attention(a["q"], a["qs"], a["pool"], a["nb"], a["out"], a["os"], a["bt"], a["mnb"],
                                    a["work"], a["nw"], a["tiles"], a["nt"], a["rpo"], a["nr"], a["split"], a["ns"],
                                    a["mpr"], a["pt"], a["tp"], a["hq"], a["hkv"], a["d"], a["bs"], a["scale"],
                                    a["dt"], a["kn"], a["ks"], a["vn"], a["vs"], a["ws"], a["wsb"], None,
                                    a["rc"], a["rs"], a["rmax"], None)

    assert call(d=96) == _lib.TB_ERR_UNSUPPORTED               # no kernel for head_dim 96
    assert call(hq=13) == _lib.TB_ERR_INVALID_ARG              # heads not a multiple of kv heads
    assert call(pt=100) == _lib.TB_ERR_INVALID_ARG             # partition not a whole number of chunks
    assert call(bs=2048, pt=256) == _lib.TB_ERR_INVALID_ARG    # partition shorter than a block
    assert call(mpr=3, ws=None) == _lib.TB_ERR_INVALID_ARG     # split rows need a workspace
    assert call(mpr=3, ws=f, wsb=100) == _lib.TB_ERR_INVALID_ARG   # ... of the right size
    assert call(pt=512) == _lib.TB_ERR_INVALID_ARG             # 16-bit kernel has a fixed partition
    assert call(kn=f, vn=None) == _lib.TB_ERR_INVALID_ARG      # fused append needs both k and v
    assert call(nw=0) == _lib.TB_OK                            # empty step: nothing to launch
    assert call(dt=0, pt=256, tiles=f, nt=1) == _lib.TB_ERR_UNSUPPORTED   # prefill tiles are 16-bit only
    assert call(tiles=None, nt=1) == _lib.TB_ERR_INVALID_ARG   # tiles announced, none given
    assert call(tiles=f, nt=1, kn=f, vn=f, ks=128, vs=128) == _lib.TB_ERR_INVALID_ARG   # fused append: decode only
    assert call(split=f, ns=1, mpr=1) == _lib.TB_ERR_INVALID_ARG   # split rows imply > 1 partition
    assert call(rc=f, rs=None, rmax=64) == _lib.TB_ERR_INVALID_ARG   # RoPE needs both tables
    assert call(rc=f, rs=f, rmax=0) == _lib.TB_ERR_INVALID_ARG       # ... and their length
    assert call(split=f, ns=3, nr=2, mpr=2, ws=f, wsb=1 << 20) == _lib.TB_ERR_INVALID_ARG   # more split rows than rows


def test_noalloc_attention_rejects_partials_beyond_its_scratch_without_launching():
    L = _lib.lib()
    f = ctypes.c_void_p(4096)
    cap = 32 << 20
    per_part = 32 * 130 * 4                    # Llama geometry: 32 heads x (128 + 2) floats
    fits, over = cap // per_part, cap // per_part + 1

    def call(tp, mpr=2, nw=2):
        return L.tb_paged_attention_noalloc(f, 4096, f, 64, f, 4096, f, 4, f, nw, None, 0, f, 2, None, 0, mpr, 256,
                                            tp, 32, 8, 128, 16, 0.0884, 2, None, 0, None, 0, None, None, None, 0,
                                            None)

    assert L.tb_paged_attention_workspace_bytes(fits, 32, 128) <= cap
    assert call(over) == _lib.TB_ERR_SCRATCH
    assert b"scratch" in L.tb_status_string(_lib.TB_ERR_SCRATCH)
    assert call(10**6) == _lib.TB_ERR_SCRATCH
    assert call(2, mpr=1, nw=0) == _lib.TB_OK                    # nothing to launch, no scratch needed


def test_workspace_size_formula():
    L = _lib.lib()
    assert L.tb_paged_attention_workspace_bytes(10, 14, 64) == 10 * 14 * 66 * 4
    assert L.tb_paged_attention_workspace_bytes(0, 14, 64) == 0
    assert L.tb_attention_partition_tokens(1, 64) == 256          # 16-bit kernel: fixed partition


def test_copy_rejects_bad_arguments_without_launching():
    L = _lib.lib()
    f = ctypes.c_void_p(4096)
    assert L.tb_block_copy(f, 2, 16, f, f, 3, 100, None) == _lib.TB_ERR_INVALID_ARG   # not 16-byte blocks
    assert L.tb_block_copy(f, 2, 16, f, f, 0, 4096, None) == _lib.TB_OK
    assert L.tb_block_gather(f, 16, f, 3, f, 0, None) == _lib.TB_ERR_INVALID_ARG
    assert L.tb_block_scatter(f, f, 0, f, 3, 4096, None) == _lib.TB_ERR_INVALID_ARG   # empty pool


def test_layer_ops_reject_bad_arguments_without_launching():
    L = _lib.lib()
    f = ctypes.c_void_p(4096)
    bf16 = 2
    lp = L.tb_linear_partials
    assert lp(f, 896, f, f, 0, 4, 896, 896, bf16, None) == _lib.TB_ERR_INVALID_ARG     # no K range
    assert lp(f, 64, f, f, 3, 4, 896, 64, bf16, None) == _lib.TB_ERR_INVALID_ARG       # 3 ranges of 2 k-slices
    assert lp(f, 896, f, f, 4, 65, 896, 896, bf16, None) == _lib.TB_ERR_UNSUPPORTED    # more than 64 rows
    assert lp(f, 896, f, f, 4, 4, 896, 896, 0, None) == _lib.TB_ERR_UNSUPPORTED        # fp32
    assert lp(f, 896, f, None, 4, 4, 896, 896, bf16, None) == _lib.TB_ERR_INVALID_ARG  # no output
    assert lp(None, 896, None, None, 4, 0, 896, 896, bf16, None) == _lib.TB_OK         # zero rows
    ls = L.tb_linear_silu_mul
    assert ls(f, 896, f, f, 4864, 4, 4856, 896, bf16, None) == _lib.TB_ERR_UNSUPPORTED  # d_ff % 16
    assert ls(f, 896, f, f, 100, 4, 4864, 896, bf16, None) == _lib.TB_ERR_INVALID_ARG   # short output rows
    assert ls(ctypes.c_void_p(4104), 896, f, f, 4864, 4, 4864, 896, bf16, None) == _lib.TB_ERR_INVALID_ARG
    rp = L.tb_rms_norm_partials
    assert rp(f, 3, None, 0, f, f, 896, 4, 896, 1e-6, bf16, None) == _lib.TB_ERR_UNSUPPORTED      # 3 splits
    assert rp(f, 4, None, 0, f, f, 900, 4, 900, 1e-6, bf16, None) == _lib.TB_ERR_UNSUPPORTED      # dim % 8
    assert rp(f, 4, None, 0, f, f, 896, 4, 896, 1e-6, 0, None) == _lib.TB_ERR_UNSUPPORTED         # fp32
    assert rp(f, 4, f, 900, f, f, 896, 4, 896, 1e-6, bf16, None) == _lib.TB_ERR_INVALID_ARG       # residual stride
    assert rp(ctypes.c_void_p(4100), 4, None, 0, f, f, 896, 4, 896, 1e-6, bf16, None) == _lib.TB_ERR_INVALID_ARG
    assert rp(None, 4, None, 0, None, None, 896, 0, 896, 1e-6, bf16, None) == _lib.TB_OK
    la = L.tb_linear_argmax
    need = L.tb_linear_argmax_workspace_bytes(4, 151936)
    assert need == 4 * 9496 * 8
    assert la(f, 896, f, 4, 151936, 896, f, need - 8, f, bf16, None) == _lib.TB_ERR_INVALID_ARG   # short workspace
    assert la(f, 896, f, 4, 151936, 896, ctypes.c_void_p(4100), need, f, bf16, None) == _lib.TB_ERR_INVALID_ARG
    assert la(f, 896, f, 4, 151936, 896, f, need, None, bf16, None) == _lib.TB_ERR_INVALID_ARG    # no ids
    assert la(f, 896, f, 4, 151930, 896, f, need, f, bf16, None) == _lib.TB_ERR_UNSUPPORTED      # N % 16
    assert la(None, 896, None, 0, 151936, 896, None, 0, None, bf16, None) == _lib.TB_OK


def test_merged_attention_refuses_rows_of_more_than_255_partitions_without_launching():
    """tb_paged_attention_merged counts a row's partitions in 8-bit per-XCD fields of its
    arrival word: 256 or more partitions of one row are refused before any launch (the
    combine kernel of tb_paged_attention serves them)."""
    L = _lib.lib()
    f = ctypes.c_void_p(4096)
    a128 = ctypes.c_void_p(1 << 20)                    # 128-byte aligned stand-in for the counters

    def call(mpr):
        tp = 2 * mpr
        wsb = L.tb_paged_attention_workspace_bytes(tp, 14, 64)
        return L.tb_paged_attention_merged(f, 896, f, 1 << 16, f, 896, f, 4096, f, tp, f, 2, mpr, 256, tp,
                                           14, 2, 64, 16, 0.125, 1, None, 0, None, 0, f, wsb,
                                           f, 8 * tp * 2, a128, 256, f, None, None, 0, None)

    assert call(256) == _lib.TB_ERR_UNSUPPORTED
    assert call(1000) == _lib.TB_ERR_UNSUPPORTED
    # the slot-map builders refuse such steps the same way
    import numpy as np
    items = np.array([[0, 0, p, 256 * 300] for p in range(300)], dtype=np.int32)
    vp = lambda x: x.ctypes.data_as(ctypes.c_void_p)
    assert L.tb_xcd_slot_map_slots(vp(items), 300, 2, 8) == _lib.TB_ERR_UNSUPPORTED
    out = np.zeros(4096, dtype=np.int32)
    assert L.tb_build_xcd_slot_map(vp(items), 300, 2, 8, vp(out), 4096) == _lib.TB_ERR_UNSUPPORTED
    assert L.tb_xcd_slot_map_slots(vp(items[:255]), 255, 2, 8) > 0
