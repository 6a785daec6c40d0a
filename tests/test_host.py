"""Host-side checks that need no GPU.

* The C-ABI library loads and exports every function `include/gpa_mi355x.h`
  declares; argument validation returns the documented error codes before
  any device work.
* The product's host logic (`merging.merge.dst_mask`, `num_dst_tokens`)
  agrees with the oracle's step-by-step restatement of merging/merge.py.
* The Python entry points refuse CPU tensors loudly (there is no CPU path).
"""
import ctypes
import re
from pathlib import Path

import pytest
import torch

from merging import _native
from merging.merge import dst_mask, num_dst_tokens, token_merge_bipartite2d
from merging.merge import fast_similarity_chunks as merge_fast_similarity_chunks
from merging.fused_similarity import fused_similarity_argmax
from merging.fused_attention import attention_keybias, LOG2E
from oracle.merge import build_dst_mask, window_draw

HEADER = Path(__file__).resolve().parent.parent / "include" / "gpa_mi355x.h"


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gpa_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_function():
    lib = _native.lib()
    declared = _declared_functions()
    assert declared, "no declarations parsed from the header"
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in {HEADER.name} but not exported"
    assert set(declared) == set(_native.exported_symbols())


def test_header_is_c99_and_links(tmp_path):
    """A C caller: the header compiles as C99 with warnings as errors, every
    declared function links against the built library by the header's
    prototype, and a call that fails argument validation returns the
    documented code and message without touching a GPU."""
    import shutil
    import subprocess
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("no C compiler")
    names = _declared_functions()
    src = tmp_path / "abi.c"
    src.write_text(
        "#include <stdio.h>\n#include \"gpa_mi355x.h\"\n"
        "int main(void) {\n"
        "  typedef void (*fn_t)(void);\n"
        "  const fn_t fns[] = {" + ", ".join(f"(fn_t)&{n}" for n in names) + "};\n"
        "  int rc = gpa_sim_argmax_bf16(0, 0, 0, GPA_DTYPE_F32, 0, 1, -1, 1, 128, 0, 0, 0, 0,"
        " 0, 0, 0, 0, 0);\n"
        "  printf(\"%d %d %d %s\\n\", gpa_abi_version(), GPA_ABI_VERSION, rc,"
        " gpa_last_error());\n"
        "  return fns[0] == 0;\n}\n")
    lib_dir = _native.LIB_PATH.parent
    exe = tmp_path / "abi"
    subprocess.run([gcc, "-std=c99", "-Wall", "-Wextra", "-Werror", "-pedantic", f"-I{HEADER.parent}",
                    str(src), "-o", str(exe), f"-L{lib_dir}", "-lgpa_mi355x",
                    f"-Wl,-rpath,{lib_dir}", "-Wl,-rpath,/opt/rocm/lib"],
                   check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    assert int(out[0]) == int(out[1]) == _native.ABI_VERSION
    assert int(out[2]) == _native.GPA_E_INVALID
    assert "negative" in " ".join(out[3:])
    # The C example of the integration guide compiles and links as written.
    doc = (HEADER.parent.parent / "INTEGRATION.md").read_text()
    snippet = re.search(r"```c\n(.*?)```", doc, re.S).group(1)
    (tmp_path / "doc.c").write_text(snippet + "\nint main(void) { return 0; }\n")
    subprocess.run([gcc, "-std=c99", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__",
                    "-I/opt/rocm/include", f"-I{HEADER.parent}", str(tmp_path / "doc.c"),
                    "-o", str(tmp_path / "doc"), f"-L{lib_dir}", "-lgpa_mi355x",
                    "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib"],
                   check=True, capture_output=True, text=True)


def test_probe_library_exports_its_entry_points():
    """The benchmark's register-only MFMA probes (a library of their own,
    not part of the product ABI): the three entry points load, argument
    errors return -1 before any launch, and the FLOP count is the
    documented one."""
    probe = _native.LIB_PATH.parent / "libgpa_probe.so"
    if not probe.exists():
        pytest.skip("probe library not built")
    lib = ctypes.CDLL(str(probe))
    lib.gpa_probe_flops.restype = ctypes.c_double
    lib.gpa_probe_flops.argtypes = [ctypes.c_int, ctypes.c_int]
    lib.gpa_probe_mfma_mix.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int64,
                                       ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    assert lib.gpa_probe_threads() == 512 * 256
    assert lib.gpa_probe_flops(0, 10) == 512 * 4 * 10 * 8 * 32768
    assert lib.gpa_probe_flops(2, 3) == 512 * 4 * 4 * 16 * 32768     # pairs of tiles
    assert lib.gpa_probe_mfma_mix(3, 1, 1, 1, 1, None) == -1
    assert lib.gpa_probe_mfma_mix(0, None, 1, 1, 1, None) == -1
    assert lib.gpa_probe_mfma_mix(0, 1, 1, 1, 0, None) == -1


def test_abi_version_and_empty_error():
    lib = _native.lib()
    assert lib.gpa_abi_version() == _native.ABI_VERSION
    assert lib.gpa_last_error() in (b"",) or isinstance(lib.gpa_last_error(), bytes)


FAKE = 4096  # a 16-byte aligned non-null address; validation returns before any use


def _sim(**kw):
    args = dict(a=FAKE, b=FAKE, out_max=FAKE, max_dtype=0, out_idx=FAKE, B=1, M=10, N=10, D=128,
                a_sb=1280, a_sm=128, b_sb=1280, b_sn=128, omax_sb=10, oidx_sb=10,
                ws=None, ws_bytes=0, stream=None)
    args.update(kw)
    return _native.lib().gpa_sim_argmax_bf16(*args.values())


@pytest.mark.parametrize("kw,code", [
    (dict(M=-1), _native.GPA_E_INVALID),
    (dict(N=0), _native.GPA_E_INVALID),
    (dict(a=None), _native.GPA_E_INVALID),
    (dict(D=48), _native.GPA_E_UNSUPPORTED),
    (dict(D=4128, a_sm=4128, b_sn=4128), _native.GPA_E_UNSUPPORTED),
    (dict(a_sm=100), _native.GPA_E_INVALID),
    (dict(a=FAKE + 2), _native.GPA_E_INVALID),
    (dict(max_dtype=5), _native.GPA_E_INVALID),
    (dict(M=100_000, N=100_000), _native.GPA_E_WORKSPACE),
])
def test_sim_argmax_argument_errors(kw, code):
    assert _sim(**kw) == code
    assert _native.lib().gpa_last_error()


def test_sim_argmax_empty_problem_is_a_no_op():
    assert _sim(M=0) == _native.GPA_OK
    assert _sim(B=0) == _native.GPA_OK


def test_workspace_bytes():
    lib = _native.lib()
    assert lib.gpa_sim_argmax_workspace_bytes(1, 10, 10, 128) == 0
    big = lib.gpa_sim_argmax_workspace_bytes(1, 75_000, 25_000, 128)
    assert big > 0 and big % 8 == 0
    assert big >= 75_000 * 8                          # one (max, idx) pair per row and split
    # 75,000 x 25,000 on 256 CUs: 8 splits of 3,136 rows (293 x 8 = 4 rounds
    # of 512 workgroups + 296), and the last 37 source blocks (9,464 rows)
    # cut into 3 sub-ranges per split: 8 x 3 more (max, idx) keys per tail row
    assert big == 8 * 75_000 * 8 + 8 * 3 * 9_464 * 8
    # 200 frames: 813 x 8 = 12 rounds + 360 items: the last 45 blocks (11,347
    # rows) halved
    assert lib.gpa_sim_argmax_workspace_bytes(1, 207_955, 66_845, 128) == \
        8 * 207_955 * 8 + 8 * 2 * 11_347 * 8
    # D = 1024 (256 x 256 tiles): 200 frames have 262 tiles of 256
    # destination rows, split 64 ways (8 per XCD, 4-5 tiles each);
    # 75,000 x 25,000 (98 tiles) 32 ways; N < 256 runs the 128 x 128 kernel
    # without splits here
    assert lib.gpa_sim_argmax_workspace_bytes(1, 207_955, 66_845, 1024) == 8 * 207_955 * 64
    assert lib.gpa_sim_argmax_workspace_bytes(1, 75_000, 25_000, 1024) == 8 * 75_000 * 32
    assert lib.gpa_sim_argmax_workspace_bytes(1, 300, 200, 1024) == 0


def _attn(**kw):
    args = dict(q=FAKE, k=FAKE, v=FAKE, bias=None, bias_kind=0, bsb=0, bsh=0, bsn=0,
                o=FAKE, lse=None, B=1, H=2, M=10, N=10, D=64,
                qsb=1280, qsh=640, qsm=64, ksb=1280, ksh=640, ksn=64,
                vsb=1280, vsh=640, vsn=64, osb=1280, osh=640, osm=64, lsb=0, lsh=0,
                ws=FAKE, ws_bytes=1 << 20, scale=0.125, stream=None)
    args.update(kw)
    return _native.lib().gpa_attn_keybias_bf16(*args.values())


@pytest.mark.parametrize("kw,code", [
    (dict(H=-1), _native.GPA_E_INVALID),
    (dict(N=0), _native.GPA_E_INVALID),
    (dict(D=48), _native.GPA_E_UNSUPPORTED),                # not a power of two
    (dict(D=512, qsm=512, ksn=512, vsn=512, osm=512), _native.GPA_E_UNSUPPORTED),
    (dict(D=8), _native.GPA_E_UNSUPPORTED),
    (dict(q=None), _native.GPA_E_INVALID),
    (dict(bias_kind=7), _native.GPA_E_INVALID),
    (dict(bias_kind=1), _native.GPA_E_INVALID),      # bias kind without a pointer
    (dict(scale=0.0), _native.GPA_E_INVALID),
    (dict(scale=float("nan")), _native.GPA_E_INVALID),
    (dict(qsm=63), _native.GPA_E_INVALID),
    (dict(k=FAKE + 8), _native.GPA_E_INVALID),
    (dict(B=70_000), _native.GPA_E_UNSUPPORTED),
    (dict(ws=None), _native.GPA_E_WORKSPACE),
    (dict(ws_bytes=16), _native.GPA_E_WORKSPACE),
    (dict(v=FAKE + 8), _native.GPA_E_INVALID),
])
def test_attn_argument_errors(kw, code):
    assert _attn(**kw) == code
    assert _native.lib().gpa_last_error()


def test_attn_empty_problem_is_a_no_op():
    assert _attn(M=0) == _native.GPA_OK


def test_attn_noalloc_refuses_shapes_beyond_the_scratch():
    """The size check of the allocation-free entry point comes before any
    HIP call, so it is a host test: 64 heads x 2^20 keys need ~300 MB of
    tile records, more than the static scratch holds."""
    lib = _native.lib()
    B, H, M, N = 1, 64, 256, 1 << 20
    assert lib.gpa_attn_keybias_workspace_bytes(B, H, M, N) > _native.NOALLOC_SCRATCH_BYTES
    rc = lib.gpa_attn_keybias_bf16_noalloc(
        FAKE, FAKE, FAKE, None, 0, 0, 0, 0, FAKE, None, B, H, M, N, 64,
        0, M * 64, 64, 0, N * 64, 64, 0, N * 64, 64, 0, M * 64, 64, 0, 0, 0.125, None)
    assert rc == _native.GPA_E_UNSUPPORTED
    assert b"static scratch" in lib.gpa_last_error()
    # the largest 200-frame workloads fit: 16 heads x 219,840 keys (core
    # blocks) and the own-frame call (3,200 batch-heads x 1,369 keys)
    assert lib.gpa_attn_keybias_workspace_bytes(1, 16, 274_800, 219_840) <= \
        _native.NOALLOC_SCRATCH_BYTES
    assert lib.gpa_attn_keybias_workspace_bytes(200, 16, 1374, 1369) <= \
        _native.NOALLOC_SCRATCH_BYTES


def test_attn_workspace_bytes():
    lib = _native.lib()
    # per (batch, head): one 144-byte record per 32-key tile, 16 bytes of row
    # bounds, and one flag byte per wave (4 waves per 256 queries)
    assert lib.gpa_attn_keybias_workspace_bytes(1, 16, 274_800, 68_700) == \
        16 * 2147 * 144 + 16 * 16 + 16 * 1074 * 4
    assert lib.gpa_attn_keybias_workspace_bytes(2, 3, 256, 32) == 6 * 144 + 6 * 16 + 6 * 4
    assert lib.gpa_attn_keybias_workspace_bytes(2, 3, 257, 33) == 6 * 2 * 144 + 6 * 16 + 6 * 8
    assert lib.gpa_attn_keybias_workspace_bytes(0, 3, 10, 33) == 0


def _merge(**kw):
    args = dict(t=FAKE, dtype=0, out=FAKE, offsets=FAKE, tokens=FAKE, B=1, H=2, N=10, S=4, D=64,
                tsb=1280, tsh=640, tsn=64, osb=512, osh=256, osn=64, mode=1, size=None,
                log_size=None, stream=None)
    args.update(kw)
    return _native.lib().gpa_merge_heads(*args.values())


@pytest.mark.parametrize("kw,code", [
    (dict(N=-1), _native.GPA_E_INVALID),
    (dict(offsets=None), _native.GPA_E_INVALID),
    (dict(mode=5), _native.GPA_E_INVALID),
    (dict(dtype=9), _native.GPA_E_INVALID),
    (dict(D=62, tsn=62, osn=62), _native.GPA_E_INVALID),     # D not a multiple of 4
    (dict(tsn=66), _native.GPA_E_INVALID),                   # misaligned row stride
    (dict(t=FAKE + 4), _native.GPA_E_INVALID),               # misaligned base (fp32)
    (dict(B=1 << 20, S=1 << 12), _native.GPA_E_UNSUPPORTED),
])
def test_merge_argument_errors(kw, code):
    assert _merge(**kw) == code
    assert _native.lib().gpa_last_error()


def test_merge_empty_is_a_no_op():
    assert _merge(B=0) == _native.GPA_OK
    assert _merge(S=0) == _native.GPA_OK


def _qk(f16=False, **kw):
    args = dict(qkv=FAKE, B=1, N=10, H=2, D=64, sb=3840, sn=384, koff=128, w=FAKE, b=FAKE,
                eps=1e-5, pos=FAKE, period=5, cs=FAKE, npos=8, q=FAKE, qd=2 if f16 else 1,
                k=FAKE, kd=0, stream=None)
    args.update(kw)
    fn = _native.lib().gpa_qk_norm_rope_f16 if f16 else _native.lib().gpa_qk_norm_rope_bf16
    return fn(*args.values())


@pytest.mark.parametrize("kw,code", [
    (dict(N=-1), _native.GPA_E_INVALID),
    (dict(D=128), _native.GPA_E_UNSUPPORTED),
    (dict(w=None), _native.GPA_E_INVALID),
    (dict(q=None), _native.GPA_E_INVALID),
    (dict(cs=None), _native.GPA_E_INVALID),                 # rotation without a table
    (dict(period=0), _native.GPA_E_INVALID),
    (dict(npos=0), _native.GPA_E_INVALID),
    (dict(qd=2), _native.GPA_E_UNSUPPORTED),                # fp16 output
    (dict(sn=380), _native.GPA_E_INVALID),                  # misaligned row stride
    (dict(koff=64), _native.GPA_E_INVALID),                 # k overlapping q
    (dict(qkv=FAKE + 8), _native.GPA_E_INVALID),            # misaligned base
])
def test_qk_norm_rope_argument_errors(kw, code):
    assert _qk(**kw) == code
    assert _native.lib().gpa_last_error()


@pytest.mark.parametrize("kw,code", [
    (dict(qd=1), _native.GPA_E_UNSUPPORTED),                # bf16 output from the fp16 entry
    (dict(kd=1), _native.GPA_E_UNSUPPORTED),
    (dict(D=32), _native.GPA_E_UNSUPPORTED),
    (dict(sn=380), _native.GPA_E_INVALID),
])
def test_qk_norm_rope_f16_argument_errors(kw, code):
    assert _qk(f16=True, **kw) == code
    assert b"gpa_qk_norm_rope_f16" in _native.lib().gpa_last_error()


def test_qk_norm_rope_empty_is_a_no_op():
    assert _qk(B=0) == _native.GPA_OK
    assert _qk(N=0, pos=None, cs=None) == _native.GPA_OK


def _pool(**kw):
    args = dict(k=FAKE, v=FAKE, pk=FAKE, pv=FAKE, size=FAKE, assign=None, B=1, H=2, S=3, P=1374,
                pts=5, gh=37, gw=37, kp=8, D=64, ksb=0, ksh=263808, ksn=64, vsb=0, vsh=263808, vsn=64,
                stream=None)
    args.update(kw)
    return _native.lib().gpa_pool_shared_bf16(*args.values())


@pytest.mark.parametrize("kw,code", [
    (dict(S=-1), _native.GPA_E_INVALID),
    (dict(kp=0), _native.GPA_E_INVALID),
    (dict(D=128), _native.GPA_E_UNSUPPORTED),
    (dict(k=None), _native.GPA_E_INVALID),
    (dict(size=None), _native.GPA_E_INVALID),
    (dict(P=1000), _native.GPA_E_INVALID),                  # frame too short for the grid
    (dict(gh=65, gw=64, P=4165, kp=9), _native.GPA_E_UNSUPPORTED),  # 4160 patches > 4096
    (dict(gh=-1), _native.GPA_E_INVALID),
    (dict(gw=38), _native.GPA_E_INVALID),                   # 37 x 38 patches + 5 > P
    (dict(ksn=60), _native.GPA_E_INVALID),                  # misaligned k rows
    (dict(vsn=63), _native.GPA_E_INVALID),                  # misaligned v rows
    (dict(vsn=68), _native.GPA_E_INVALID),                  # v rows not 16-byte aligned
])
def test_pool_shared_argument_errors(kw, code):
    assert _pool(**kw) == code
    assert _native.lib().gpa_last_error()


def test_pool_shared_empty_is_a_no_op():
    assert _pool(B=0) == _native.GPA_OK
    assert _pool(S=0) == _native.GPA_OK
    assert _pool(gh=0) == _native.GPA_OK


def _metric(**kw):
    args = dict(x=FAKE, dt=_native.GPA_DTYPE_F32, B=1, N=5496, C=1024, sb=0, sn=1024, proj=FAKE,
                P=128, order=None, mode=0, out=FAKE, stream=None)
    args.update(kw)
    return _native.lib().gpa_merge_metric_bf16(*args.values())


@pytest.mark.parametrize("kw,code", [
    (dict(N=-1), _native.GPA_E_INVALID),
    (dict(dt=2), _native.GPA_E_UNSUPPORTED),                # fp16 metric
    (dict(mode=3), _native.GPA_E_INVALID),
    (dict(mode=2, dt=_native.GPA_DTYPE_BF16), _native.GPA_E_UNSUPPORTED),   # fp16 projection: fp32 metric
    (dict(C=1000, sn=1000), _native.GPA_E_UNSUPPORTED),     # C not in {256, 512, 768, 1024}
    (dict(P=64), _native.GPA_E_UNSUPPORTED),
    (dict(x=None), _native.GPA_E_INVALID),
    (dict(out=None), _native.GPA_E_INVALID),
    (dict(sn=1020), _native.GPA_E_INVALID),                 # rows not 16-byte aligned
])
def test_merge_metric_argument_errors(kw, code):
    assert _metric(**kw) == code
    assert _native.lib().gpa_last_error()


def test_merge_metric_empty_is_a_no_op():
    assert _metric(B=0) == _native.GPA_OK
    assert _metric(N=0) == _native.GPA_OK


def _rln(**kw):
    args = dict(x=FAKE, y=FAKE, gamma=FAKE, w=FAKE, b=FAKE, eps=1e-6, rows=10, C=1024, x_sn=1024,
                y_sn=1024, h=FAKE, h_sn=1024, ln=FAKE, ln_sn=1024, stream=None)
    args.update(kw)
    return _native.lib().gpa_residual_layernorm_bf16(*args.values())


@pytest.mark.parametrize("kw,code", [
    (dict(rows=-1), _native.GPA_E_INVALID),
    (dict(C=1000, x_sn=1000), _native.GPA_E_UNSUPPORTED),      # not a multiple of 512
    (dict(C=8192), _native.GPA_E_UNSUPPORTED),
    (dict(x=None), _native.GPA_E_INVALID),
    (dict(gamma=None), _native.GPA_E_INVALID),                  # y without gamma
    (dict(w=None), _native.GPA_E_INVALID),                      # ln_out without weight
    (dict(h=None, ln=None), _native.GPA_E_INVALID),             # no output
    (dict(y=None), _native.GPA_E_INVALID),                      # h_out without y
    (dict(eps=float("nan")), _native.GPA_E_INVALID),
    (dict(x_sn=1020), _native.GPA_E_INVALID),                   # misaligned rows
])
def test_residual_layernorm_argument_errors(kw, code):
    assert _rln(**kw) == code
    assert _native.lib().gpa_last_error()


def test_residual_layernorm_empty_is_a_no_op():
    assert _rln(rows=0) == _native.GPA_OK


@pytest.mark.parametrize("frames,w,h,sx,sy,ns,no_rand", [
    (6, 37, 37, 2, 2, 5, False), (5, 7, 5, 2, 2, 5, False), (3, 9, 9, 3, 3, 1, False),
    (4, 6, 6, 2, 2, 5, True), (1, 6, 6, 2, 2, 5, False), (3, 10, 4, 3, 2, 2, False),
])
def test_product_mask_matches_oracle(frames, w, h, sx, sy, ns, no_rand):
    g1 = torch.Generator().manual_seed(33)
    g2 = torch.Generator().manual_seed(33)
    mine = dst_mask(frames, w, h, sx, sy, ns, no_rand, g1, torch.device("cpu"))
    cell = window_draw(frames, w, h, sx, sy, g2) if frames > 1 and not no_rand else None
    ref = build_dst_mask(frames, w, h, sx, sy, ns, no_rand, cell)
    assert torch.equal(mine, ref)
    assert int((mine == -1).sum()) == num_dst_tokens(frames, w, h, sx, sy, ns, no_rand)


def test_cpu_tensors_are_refused():
    a = torch.randn(1, 8, 128)
    with pytest.raises(AssertionError):
        fused_similarity_argmax(a, a)
    q = torch.randn(1, 2, 8, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        attention_keybias(q, q, q, None, 0.125)
    with pytest.raises(ValueError):
        token_merge_bipartite2d(torch.randn(1, 2 * 41, 32), 6, 6, 2, 2, 5)
    with pytest.raises(ValueError):
        token_merge_bipartite2d(torch.randn(1, 2 * 41, 32), 6, 6, 2, 2, 0)
    with pytest.raises(AssertionError):
        merge_fast_similarity_chunks(a, a.transpose(1, 2), 5000)


def test_merge_fast_similarity_chunks_argument_errors():
    """The reference's chunked entry point keeps its argument checks: a
    non-positive chunk size (the reference's `range` step) and operands
    that are not [B, M, C] / [B, C, N]."""
    a = torch.randn(1, 8, 128)
    with pytest.raises(ValueError):
        merge_fast_similarity_chunks(a, a.transpose(1, 2), 0)
    with pytest.raises(AssertionError):
        merge_fast_similarity_chunks(a[0], a.transpose(1, 2), 5000)


def test_log2e_constant():
    import math
    assert LOG2E == pytest.approx(1.0 / math.log(2.0), abs=1e-15)


def _build_module():
    import importlib.util
    spec = importlib.util.spec_from_file_location(
        "gpa_build", Path(__file__).resolve().parent.parent / "gpa-vggt_amd" / "build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_hot_kernels_have_no_spills_or_scratch():
    """Every kernel of the similarity and attention sources (head dim 64
    and the other head dims), compiled with the library's own flags, fits
    its registers: no VGPR or SGPR spills and no scratch (hipcc's
    kernel-resource-usage report).  The head-dim-64 attention kernel and the
    tiled kernel at head dim 128 must also keep two waves per SIMD."""
    import shutil
    b = _build_module()
    if shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists():
        pytest.skip("hipcc not available")
    report = b.resource_usage(["attn_keybias.hip", "sim_argmax.hip", "attn_any_dim.hip"])
    bad = {}
    for src, kernels in report.items():
        assert kernels, f"no kernels reported for {src}"
        for name, use in kernels.items():
            if use.get("vgpr_spill") or use.get("sgpr_spill") or use.get("scratch"):
                bad[f"{src}:{name}"] = use
    assert not bad, f"kernels with spills or scratch: {bad}"
    attn = [u for n, u in report["attn_keybias.hip"].items() if "attn_main_kernel" in n]
    assert len(attn) == 2 and all(u["occupancy"] >= 2 for u in attn), attn
    tiled = [u for n, u in report["attn_any_dim.hip"].items() if "attn_tiled_kernelILi128" in n]
    assert len(tiled) == 2 and all(u["occupancy"] >= 2 for u in tiled), tiled


def test_bench_measures_one_gpu_and_prices_against_the_bf16_peak(capsys):
    """bench.py refuses N > 1 with a message (one GPU carries the whole
    path here), and a kernel entry's TFLOP/s and % of peak follow from the
    FLOP count and the time against the 2,516.6 TFLOP/s dense bf16 peak."""
    import importlib.util
    spec = importlib.util.spec_from_file_location(
        "bench_mod", Path(__file__).resolve().parent.parent / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    assert bench.main(["--gpus", "2"]) == 2
    assert "one GPU" in capsys.readouterr().err
    e = bench.kernel_entry(7.7327400960e13, 64.0)
    assert abs(e["tflops"] - 7.7327400960e13 / 64e-3 / 1e12) < 0.01
    assert abs(e["pct_peak"] - 100 * e["tflops"] / 2516.6) < 0.01
    args = bench.parse_args([])
    assert args.gpus == 1 and args.steps > 0 and args.warmup >= 0
