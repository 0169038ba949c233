"""C ABI checks that need no GPU: the library loads, exports every entry point include/exl3_grouped.h declares,
and rejects bad arguments with EXL3_ERR_ARG and a message before launching anything (the reference's
TORCH_CHECK contract, kernel/exl3_grouped_prefill.cu:288-372, kernel/exl3_fat_gemm_v2.cu:236-252)."""
import ctypes
import os
import re

import pytest
import torch

import exl3_grouped as gp
from exl3_grouped import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "exl3_grouped.h")
FAKE = ctypes.c_void_p(0x1000)        # never dereferenced: every case below fails validation first


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(exl3_\w+)\s*\(", text)))


def test_header_declares_what_the_binding_binds():
    assert declared_functions() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.exl3_abi_version() == _lib.ABI_VERSION


def rc_and_msg(name, *args):
    rc = getattr(_lib.load(), name)(*args)
    return rc, _lib.last_error()


def test_build_blocks_rejects_too_many_experts():
    rc, msg = rc_and_msg("exl3_build_blocks", FAKE, 1025, 10, FAKE, FAKE, FAKE, None)
    assert rc == _lib.EXL3_ERR_ARG and msg == "too many experts"


def test_build_tiles_rejects_bad_tile_rows():
    rc, msg = rc_and_msg("exl3_build_tiles", FAKE, 8, 96, 10, FAKE, FAKE, FAKE, None)
    assert rc == _lib.EXL3_ERR_ARG and "tile_rows" in msg


def test_row_had_rejects_bad_k():
    rc, msg = rc_and_msg("exl3_row_had", FAKE, FAKE, FAKE, FAKE, FAKE, 100, 100, 4, 100, 1, None)
    assert rc == _lib.EXL3_ERR_ARG and "multiple of 128" in msg
    rc, msg = rc_and_msg("exl3_row_had", FAKE, FAKE, FAKE, FAKE, FAKE, 256, 128, 4, 256, 1, None)
    assert rc == _lib.EXL3_ERR_ARG and "match suh" in msg


def test_act_had_rejects_bad_width():
    rc, msg = rc_and_msg("exl3_act_had", FAKE, 300, FAKE, FAKE, FAKE, 128, 4, 128, ctypes.c_float(10.0), None)
    assert rc == _lib.EXL3_ERR_ARG and "2I" in msg


def _gemm(**kw):
    a = dict(a=FAKE, a_rows=256, size_k=512, pg=FAKE, pu=None, es=32 * 16 * 64, tk=32, tn=16, bits=4, sg=FAKE,
             su=None, ss=256, be=FAKE, br=FAKE, mb=10, counts=FAKE, row0=FAKE, E=8, tok=FAKE, rw=FAKE, ri=None,
             out=FAKE, out_rows=64, mode=1)
    a.update(kw)
    return rc_and_msg("exl3_grouped_gemm", *a.values(), None)


def test_grouped_gemm_contract():
    assert _gemm(bits=5)[0] == _lib.EXL3_ERR_ARG
    assert "K mismatch" in _gemm(size_k=500)[1]
    assert "K mismatch" in _gemm(size_k=480, tk=30)[1]                 # K % 64
    assert "multiple of 128" in _gemm(tn=12)[1]
    assert "too many experts" in _gemm(E=2000)[1]
    assert "single tensor" in _gemm(pu=FAKE, su=FAKE)[1]
    assert "gate/up strides must match" in _gemm(pu=FAKE, su=None)[1]
    assert "mode must be" in _gemm(mode=5)[1]
    assert "mode 4: T16" in _gemm(mode=4, a_rows=250, out_rows=250)[1]   # T16 rows round up to 256
    assert "mode 3: out fp32" in _gemm(mode=3)[1]                       # out_rows < a_rows
    assert "route_index" in _gemm(mode=2)[1]
    assert "combine" in rc_and_msg("exl3_combine_routes", FAKE, FAKE, None, 4, 8, 10, 8, 6, None)[1]
    assert "topk above 32" in rc_and_msg("exl3_combine_routes", FAKE, FAKE, None, 4, 8, 10, 33, 8, None)[1]
    assert "fp32, bf16 or fp16" in rc_and_msg("exl3_combine_routes_dt", FAKE, FAKE, _lib.DTYPE_I32, None, 4, 8, 10, 8,
                                              8, None)[1]
    assert "aligned" in rc_and_msg("exl3_combine_routes_dt", FAKE, ctypes.c_void_p(0x1004), _lib.DTYPE_BF16, None, 4, 8, 10, 8, 8,
                                   None)[1]
    a = dict(a=FAKE, a_rows=256, size_k=512, a_layout=0, pg=FAKE, pu=None, es=32 * 16 * 64, tk=32, tn=16, bits=4,
             sg=FAKE, su=None, ss=256, be=FAKE, br=FAKE, mb=10, tile_rows=96, counts=FAKE, row0=FAKE, E=8, tok=FAKE,
             rw=FAKE, ri=None, out=FAKE, out_rows=64, mode=1)
    assert "tile_rows" in rc_and_msg("exl3_grouped_gemm_ex", *a.values(), None)[1]
    a.update(tile_rows=256, a_layout=2)
    assert "layout" in rc_and_msg("exl3_grouped_gemm_ex", *a.values(), None)[1]
    assert "layout" in rc_and_msg("exl3_row_had_ex", FAKE, FAKE, FAKE, FAKE, FAKE, 256, 256, 4, 256, 1, 5, None)[1]


def test_fat_gemm_contract():
    args = dict(a=FAKE, m=300, k=4096, pk=FAKE, tk=256, tn=96, words=64, out=FAKE, out_rows=300, svh=FAKE,
                svh_len=1536, bits=4, mcg=1, mul1=0, variant=1)

    def call(**kw):
        a = dict(args)
        a.update(kw)
        return rc_and_msg("exl3_fat_gemm", *a.values(), None)

    assert "MCG" in call(mcg=0)[1] and "MCG" in call(mul1=1)[1] and "MCG" in call(bits=5)[1]
    assert "does not match packed" in call(k=4000)[1]
    assert "svh N dimension" in call(svh_len=1024)[1]
    assert "16*K" in call(words=48)[1]
    assert "unknown variant" in call(variant=4)[1]
    assert "out shape" in call(out_rows=299)[1]
    lib = _lib.load()
    # per-variant LDS of the kernels each schedule launches: 4-wave kernels (64/256-row tiles) stage 4 waves x 16 rows
    # x 132 floats for the scatter, the 8-wave kernel (512-row tiles, also picked by variant 1) 8 waves' worth
    assert [lib.exl3_smem_bytes(v) for v in range(4)] == [4 * 16 * 132 * 4, 8 * 16 * 132 * 4,
                                                          4 * 16 * 132 * 4, 8 * 16 * 132 * 4]
    assert lib.exl3_smem_bytes(9) == -1 and lib.exl3_smem_bytes(-1) == -1


def test_sort_routes_contract():
    lib = _lib.load()
    need = lib.exl3_sort_routes_workspace_bytes(100, 8, 288)
    assert need > 0
    rc, msg = rc_and_msg("exl3_sort_routes", FAKE, _lib.DTYPE_I64, FAKE, _lib.DTYPE_F32, 100, 8, 288, FAKE, FAKE, FAKE,
                         None, FAKE, FAKE, FAKE, need - 1, None)
    assert rc == _lib.EXL3_ERR_ARG and "workspace" in msg
    rc, msg = rc_and_msg("exl3_sort_routes", FAKE, _lib.DTYPE_F32, FAKE, _lib.DTYPE_F32, 100, 8, 288, FAKE, FAKE,
                         FAKE, None, FAKE, FAKE, FAKE, need, None)
    assert rc == _lib.EXL3_ERR_ARG and "int64 or int32" in msg


def test_decode_and_reconstruct_contract():
    assert "even" in rc_and_msg("exl3_decode_states", FAKE, FAKE, 3, None)[1]
    assert "MCG" in rc_and_msg("exl3_reconstruct", FAKE, FAKE, 2, 2, 4, 1, 1, None)[1]


# ------------------------------------------------------------------------------------------- torch shim
def test_shim_checks_dtypes_before_device():
    c = torch.zeros(8, dtype=torch.int64)
    with pytest.raises(RuntimeError, match="int32 tensors"):
        gp.build_blocks(c, c, c, c)
    i32 = torch.zeros(8, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="tensors must be CUDA"):
        gp.build_blocks(i32, torch.zeros(20, dtype=torch.int32), torch.zeros(20, dtype=torch.int32),
                        torch.zeros(2, dtype=torch.int32))


def test_shim_fat_gemm_messages():
    a = torch.zeros(300, 4096, dtype=torch.float16)
    pk = torch.zeros(256, 96, 64, dtype=torch.int16)
    out = torch.zeros(300, 1536)
    svh = torch.zeros(1536, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="only K2/K3/K4 MCG tensors"):
        gp.fat_gemm_v2(a, pk, out, svh, 4, False, False, 1)
    with pytest.raises(RuntimeError, match="a must be float16"):
        gp.fat_gemm_v2(a.float(), pk, out, svh, 4, True, False, 1)
    with pytest.raises(RuntimeError, match="unknown variant"):
        gp.fat_gemm_v2(a, pk, out, svh, 4, True, False, 7)
    with pytest.raises(RuntimeError, match="tensors must be CUDA"):
        gp.fat_gemm_v2(a, pk, out, svh, 4, True, False, 1)
    assert gp.smem_bytes(5) == -1
    # PR77's names and argument order (kernel/test_fat_v2.py:122,134), same checks before the device
    with pytest.raises(RuntimeError, match="only K2/K3/K4 MCG tensors"):
        gp.exl3_fat_gemm(a, pk, out, svh, 4, False, False)
    with pytest.raises(RuntimeError, match="tensors must be CUDA"):
        gp.exl3_fat_gemm(a, pk, out, svh, 4, True, False)
    tok = torch.zeros(300, dtype=torch.int64)
    rw = torch.zeros(300, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="routing dtypes"):
        gp.exl3_fat_gemm_scatter(a, pk, out, svh, tok, rw.float(), 4, True, False)
    with pytest.raises(RuntimeError, match="tensors must be CUDA"):
        gp.exl3_fat_gemm_scatter(a, pk, out, svh, tok, rw, 4, True, False)


def test_shim_grouped_gemm_messages():
    a = torch.zeros(256, 512, dtype=torch.float16)
    w13 = torch.zeros(8, 2, 32, 16, 64, dtype=torch.int16)
    svh = torch.zeros(8, 2, 256, dtype=torch.float16)
    i32 = torch.zeros(20, dtype=torch.int32)
    gu = torch.zeros(256, 512, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="a fp16 contiguous"):
        gp.grouped_gemm(a.float(), w13[:, 0], w13[:, 1], svh[:, 0], svh[:, 1], i32, i32, i32[:8], i32[:8], None,
                        None, gu, 0)
    with pytest.raises(RuntimeError, match="mode 0"):
        gp.grouped_gemm(a, w13[:, 0], w13[:, 1], svh[:, 0], svh[:, 1], i32, i32, i32[:8], i32[:8], None, None,
                        gu[:, :256], 0)
    with pytest.raises(RuntimeError, match="tensors must be CUDA"):
        gp.grouped_gemm(a, w13[:, 0], w13[:, 1], svh[:, 0], svh[:, 1], i32, i32, i32[:8], i32[:8], None, None,
                        gu, 0)


def test_linear_contract():
    args = dict(x=FAKE, m=300, k=4096, pk=FAKE, tk=256, tn=96, bits=4, suh=FAKE, svh=FAKE, work=FAKE, out=FAKE,
                dtype=1)                         # EXL3_DTYPE_F16

    def call(**kw):
        a = dict(args)
        a.update(kw)
        return rc_and_msg("exl3_linear", a["x"], a["m"], a["k"], a["pk"], a["tk"], a["tn"], a["bits"], a["suh"],
                          a["svh"], a["work"], a["out"], a["dtype"], None)

    rc, msg = call(bits=5)
    assert rc == _lib.EXL3_ERR_ARG and "bits" in msg
    rc, msg = call(k=4000, tk=250)
    assert rc == _lib.EXL3_ERR_ARG and "multiple of 128" in msg
    rc, msg = call(tn=95)
    assert rc == _lib.EXL3_ERR_ARG and "N must be a multiple of 128" in msg
    rc, msg = call(dtype=4)
    assert rc == _lib.EXL3_ERR_ARG and "fp32 or fp16" in msg
    rc, msg = call(x=None)
    assert rc == _lib.EXL3_ERR_ARG and msg == "null pointer"
    rc, msg = call(m=0, x=None)                      # nothing to do: no pointer is needed
    assert rc == _lib.EXL3_OK
    assert _lib.load().exl3_linear_workspace_bytes(300, 4096) == 304 * 4096 * 2
    assert _lib.load().exl3_linear_workspace_bytes(-1, 4096) == -1


def test_route_topk_contract():
    def call(E=288, k=8, ldt=0, idt=4, T=10, ld=288, logits=FAKE):
        return rc_and_msg("exl3_route_topk", logits, ldt, ld, None, T, E, k, 1, ctypes.c_float(2.5), FAKE, idt,
                          FAKE, None)
    rc, msg = call(E=1025)
    assert rc == _lib.EXL3_ERR_ARG and msg == "too many experts"
    rc, msg = call(k=17)
    assert rc == _lib.EXL3_ERR_ARG and "topk" in msg
    rc, msg = call(E=4, k=5)
    assert rc == _lib.EXL3_ERR_ARG and "topk" in msg
    rc, msg = call(ldt=3)
    assert rc == _lib.EXL3_ERR_ARG and "logits" in msg
    rc, msg = call(idt=0)
    assert rc == _lib.EXL3_ERR_ARG and "int64 or int32" in msg
    rc, msg = call(ld=100)
    assert rc == _lib.EXL3_ERR_ARG and msg == "bad sizes"
    rc, msg = call(logits=None)
    assert rc == _lib.EXL3_ERR_ARG and msg == "null pointer"
    rc, msg = call(T=0, logits=None)
    assert rc == _lib.EXL3_OK


def test_split_gemm_contract():
    args = dict(a=FAKE, a_rows=256, size_k=512, a_layout=1, pg=FAKE, pu=None, es=32 * 16 * 64, tk=32, tn=16, bits=4,
                sg=FAKE, su=None, ss=256, be=FAKE, br=FAKE, mb=10, tile_rows=128, counts=FAKE, row0=FAKE, E=8,
                tok=FAKE, rw=FAKE, ri=None, out=FAKE, out_rows=256, mode=1, k_split=2)

    def call(**kw):
        a = dict(args)
        a.update(kw)
        return rc_and_msg("exl3_grouped_gemm_split", *a.values(), None)

    for ks in (0, 9):                                    # K = 512: 16 stages, at most 8 slices of 2
        rc, msg = call(k_split=ks)
        assert rc == _lib.EXL3_ERR_ARG and "k_split" in msg
    rc, msg = call(mode=0, k_split=2)
    assert rc == _lib.EXL3_ERR_ARG and "accumulating mode" in msg
    rc, msg = call(mode=3, tile_rows=512)
    assert rc == _lib.EXL3_ERR_ARG and "mode 3" in msg
    rc, msg = call(mode=5, k_split=1)
    assert rc == _lib.EXL3_ERR_ARG and "mode must be" in msg
    # the launch that also clears a buffer: the clear's contract is checked before anything runs
    for zero, n, mb, text in ((None, 8, 10, "zero must be"), (FAKE, 6, 10, "zero must be"),
                              (ctypes.c_void_p(0x1004), 8, 10, "zero must be"), (FAKE, -4, 10, "zero must be"),
                              (FAKE, 8, 0, "max_blocks")):
        a = dict(args)
        a.update(mb=mb, k_split=1)
        rc, msg = rc_and_msg("exl3_grouped_gemm_clear", *a.values(), zero, n, None)
        assert rc == _lib.EXL3_ERR_ARG and text in msg, (zero, n, mb, msg)
    rc, msg = rc_and_msg("exl3_act_had_f32", FAKE, 300, FAKE, FAKE, FAKE, 128, 4, 128, ctypes.c_float(10.0), None)
    assert rc == _lib.EXL3_ERR_ARG and "2I" in msg


DECODE_ARGS = dict(x=FAKE, tokens=4, hidden=4096, ids=FAKE, ids_dt=4, w=FAKE, w_dt=0, topk=8, E=288, inter=768,
                   bits=4, pg=FAKE, pu=FAKE, es13=2 * 256 * 48 * 64, suh=FAKE, suh_s=8192, svg=FAKE, svu=FAKE,
                   sv_s=1536, pd=FAKE, es2=48 * 256 * 64, suhd=FAKE, suhd_s=768, svd=FAKE, svd_s=4096,
                   limit=ctypes.c_float(10.0), out=ctypes.c_void_p(0x2000), ws=ctypes.c_void_p(0x10000), ws_bytes=0)


def decode_call(**kw):
    a = dict(DECODE_ARGS)
    a.update(kw)
    return rc_and_msg("exl3_moe_decode", *a.values(), None)


def test_moe_decode_contract():
    lib = _lib.load()
    need = lib.exl3_moe_decode_workspace_bytes(4, 8, 288, 4096, 768)
    R, r16 = 32, 32
    regions = [R * 8, R * 2, R * 4, 288 * 4, 288 * 4, (32 + 0) * 4, (32 + 0) * 4, 8, r16 * 4096 * 2, R * 1536 * 4,
               r16 * 768 * 2]
    assert need % 256 == 0 and need >= sum(regions) + lib.exl3_sort_routes_workspace_bytes(4, 8, 288)
    assert lib.exl3_moe_decode_workspace_bytes(8, 8, 288, 4096, 768) > need
    assert lib.exl3_moe_decode_workspace_bytes(-1, 8, 288, 4096, 768) == -1
    assert lib.exl3_moe_decode_workspace_bytes(4, 8, 2000, 4096, 768) == -1
    rc, msg = decode_call(hidden=4000)
    assert rc == _lib.EXL3_ERR_ARG and "multiples of 128" in msg
    rc, msg = decode_call(bits=5)
    assert rc == _lib.EXL3_ERR_ARG and "bits" in msg
    rc, msg = decode_call(E=2000)
    assert rc == _lib.EXL3_ERR_ARG and msg == "too many experts"
    rc, msg = decode_call(x=None)
    assert rc == _lib.EXL3_ERR_ARG and msg == "null pointer"
    rc, msg = decode_call(out=ctypes.c_void_p(0x2004))
    assert rc == _lib.EXL3_ERR_ARG and "aligned" in msg
    rc, msg = decode_call(ws_bytes=need - 1)
    assert rc == _lib.EXL3_ERR_ARG and "workspace too small" in msg
    rc, msg = decode_call(tokens=0, x=None, ids=None, w=None, out=None, ws=None)
    assert rc == _lib.EXL3_OK                            # nothing to do: no pointer is needed


def test_moe_decode_noalloc_contract():
    """The no-allocation decode entry point rejects a call whose workspace would not fit its fixed 32 MiB scratch
    before touching a GPU, and an empty batch is a no-op."""
    lib = _lib.load()
    assert lib.exl3_moe_decode_workspace_bytes(256, 8, 288, 4096, 768) <= 32 << 20
    assert lib.exl3_moe_decode_workspace_bytes(512, 8, 288, 4096, 768) > 32 << 20
    args = [FAKE, 512, 4096, FAKE, _lib.DTYPE_I64, FAKE, _lib.DTYPE_F32, 8, 288, 768, 4, FAKE, FAKE, 1, FAKE, 1,
            FAKE, FAKE, 1, FAKE, 1, FAKE, 1, FAKE, 1, ctypes.c_float(10.0), FAKE, None]
    rc, msg = rc_and_msg("exl3_moe_decode_noalloc", *args)
    assert rc == _lib.EXL3_ERR_ARG and "scratch" in msg
    args[1] = 0
    rc, msg = rc_and_msg("exl3_moe_decode_noalloc", *args)
    assert rc == _lib.EXL3_OK


def test_shim_moe_decode_messages():
    x = torch.zeros(4, 512, dtype=torch.float16)
    ids = torch.zeros(4, 2, dtype=torch.int64)
    w = torch.zeros(4, 2)
    w13 = torch.zeros(8, 2, 32, 16, 64, dtype=torch.int16)
    w2 = torch.zeros(8, 16, 32, 64, dtype=torch.int16)
    s13, v13 = torch.zeros(8, 2, 512, dtype=torch.float16), torch.zeros(8, 2, 256, dtype=torch.float16)
    s2, v2 = torch.zeros(8, 256, dtype=torch.float16), torch.zeros(8, 512, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="contiguous fp16"):
        gp.moe_decode(x.float(), ids, w, w13, s13, v13, w2, s2, v2, 10.0)
    with pytest.raises(RuntimeError, match="topk_ids"):
        gp.moe_decode(x, ids[:3], w, w13, s13, v13, w2, s2, v2, 10.0)
    with pytest.raises(RuntimeError, match="w2_trellis"):
        gp.moe_decode(x, ids, w, w13, s13, v13, w2[:, :8], s2, v2, 10.0)
    with pytest.raises(RuntimeError, match="shapes"):
        gp.moe_decode(x, ids, w, w13, s13, v13, w2, s2[:, :128], v2, 10.0)
    with pytest.raises(RuntimeError, match="tensors must be CUDA"):
        gp.moe_decode(x, ids, w, w13, s13, v13, w2, s2, v2, 10.0,
                      workspace=torch.empty(gp.moe_decode_workspace_bytes(4, 2, 8, 512, 256), dtype=torch.uint8))


def test_route_prep_small_contract():
    def call(T=4, k=8, E=288, tr=128, mt=40, za=None, na=0, ids=FAKE):
        return rc_and_msg("exl3_route_prep_small", ids, 4, FAKE, 0, T, k, E, tr, mt, FAKE, FAKE, FAKE, FAKE, FAKE,
                          FAKE, FAKE, FAKE, za, na, None, 0, None)
    rc, msg = call(T=257)
    assert rc == _lib.EXL3_ERR_ARG and "at most 2048 routes" in msg
    rc, msg = call(tr=100)
    assert rc == _lib.EXL3_ERR_ARG and "tile_rows" in msg
    rc, msg = call(E=1025)
    assert rc == _lib.EXL3_ERR_ARG and msg == "too many experts"
    rc, msg = call(za=FAKE, na=6)
    assert rc == _lib.EXL3_ERR_ARG and "float4" in msg
    rc, msg = call(za=ctypes.c_void_p(0x1004), na=8)
    assert rc == _lib.EXL3_ERR_ARG and "aligned" in msg
    rc, msg = call(ids=None)
    assert rc == _lib.EXL3_ERR_ARG and msg == "null pointer"


def test_build_tiles_split_contract():
    rc, msg = rc_and_msg("exl3_build_tiles_split", FAKE, 8, 256, 128, 10, 8, FAKE, FAKE, FAKE, FAKE, FAKE, None, 0, None)
    assert rc == _lib.EXL3_ERR_ARG and "thin_rows 64" in msg
    rc, msg = rc_and_msg("exl3_build_tiles_split", FAKE, 8, 64, 64, 10, 8, FAKE, FAKE, FAKE, FAKE, FAKE, None, 0, None)
    assert rc == _lib.EXL3_ERR_ARG and "tile_rows" in msg
    rc, msg = rc_and_msg("exl3_build_tiles_split", FAKE, 1025, 256, 64, 10, 8, FAKE, FAKE, FAKE, FAKE, FAKE, None, 0, None)
    assert rc == _lib.EXL3_ERR_ARG and msg == "too many experts"
    rc, msg = rc_and_msg("exl3_build_tiles_split", FAKE, 8, 256, 64, 10, 8, FAKE, FAKE, None, FAKE, FAKE, None, 0, None)
    assert rc == _lib.EXL3_ERR_ARG and msg == "null pointer"
    for zero, n in ((None, 8), (FAKE, 6), (ctypes.c_void_p(0x1004), 8), (FAKE, -4)):   # the clear: NULL, ragged, misaligned
        rc, msg = rc_and_msg("exl3_build_tiles_split", FAKE, 8, 256, 64, 10, 8, FAKE, FAKE, FAKE, FAKE, FAKE, zero, n,
                             None)
        assert rc == _lib.EXL3_ERR_ARG and "zero must be" in msg, (zero, n)


def test_sort_routes_split_tiles_contract():
    """The fused preparation validates like exl3_sort_routes and exl3_build_tiles_split, before any launch."""
    need = _lib.load().exl3_sort_routes_workspace_bytes(100, 8, 288)

    def call(ids_dtype=_lib.DTYPE_I64, experts=288, ws_bytes=need, tile_rows=256, thin_rows=64, fe=FAKE, zero=None,
             n=0):
        return rc_and_msg("exl3_sort_routes_split_tiles", FAKE, ids_dtype, FAKE, _lib.DTYPE_F32, 100, 8, experts, FAKE,
                          FAKE, FAKE, None, FAKE, FAKE, FAKE, ws_bytes, tile_rows, thin_rows, 10, 8, fe, FAKE, FAKE,
                          FAKE, FAKE, zero, n, None)

    rc, msg = call(ws_bytes=need - 1)
    assert rc == _lib.EXL3_ERR_ARG and "workspace" in msg
    rc, msg = rc_and_msg("exl3_sort_routes_split_tiles", FAKE, _lib.DTYPE_I64, FAKE, _lib.DTYPE_F32, 100, 8, 288, FAKE,
                         FAKE, FAKE, None, FAKE, FAKE, ctypes.c_void_p(0x1008), need, 256, 64, 10, 8, FAKE, FAKE, FAKE,
                         FAKE, FAKE, None, 0, None)
    assert rc == _lib.EXL3_ERR_ARG and "16-byte aligned" in msg
    rc, msg = call(ids_dtype=_lib.DTYPE_F32)
    assert rc == _lib.EXL3_ERR_ARG and "int64 or int32" in msg
    rc, msg = call(experts=1025)
    assert rc == _lib.EXL3_ERR_ARG and msg == "too many experts"
    rc, msg = call(tile_rows=64)
    assert rc == _lib.EXL3_ERR_ARG and "tile_rows" in msg
    rc, msg = call(thin_rows=128)
    assert rc == _lib.EXL3_ERR_ARG and "thin_rows 64" in msg
    rc, msg = call(fe=None)
    assert rc == _lib.EXL3_ERR_ARG and msg == "null pointer"
    for zero, n in ((None, 8), (FAKE, 6), (ctypes.c_void_p(0x1004), 8), (FAKE, -4)):
        rc, msg = call(zero=zero, n=n)
        assert rc == _lib.EXL3_ERR_ARG and "zero must be" in msg, (zero, n)
