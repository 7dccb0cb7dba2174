"""C-ABI checks that need no GPU: the library loads, exports every function
include/*.h declares, and rejects bad descriptors with the documented status
codes before touching the device."""
import ctypes
import glob
import os
import re

import pytest

from servoflow_amd import abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for path in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(path).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        for m in re.finditer(r"\b(sf_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return sorted(names)


def test_header_declares_entry_points():
    names = declared_functions()
    for required in ("sf_attn_fwd", "sf_attn_workspace_bytes", "sf_strerror"):
        assert required in names


def _owner_lib(name):
    # sf_rdt_* (model runtime) and sf_safetensors_* (checkpoint reader) live
    # in libsf_rdt.so, everything else in libsf_hip_kernels.so
    if name.startswith(("sf_rdt_", "sf_safetensors_")):
        from servoflow_amd import rdt
        return rdt.lib()
    return abi.lib()


@pytest.mark.parametrize("name", declared_functions())
def test_library_exports_symbol(name):
    assert hasattr(_owner_lib(name), name), f"{name} declared in include/ but not exported"


def test_strerror_texts():
    for st in (abi.SF_OK, abi.SF_EINVAL, abi.SF_ENOTSUP, abi.SF_EWORKSPACE, abi.SF_ELAUNCH, abi.SF_EDEVICE,
               abi.SF_ESCRATCH):
        assert len(abi.strerror(st)) > 3
    assert abi.strerror(12345) == "unknown status"


def _fwd(desc, q=16, k=16, v=16, o=16, ws=None, wsn=0):
    return abi.lib().sf_attn_fwd(ctypes.byref(desc), q, k, v, o, ws, wsn, None)


def test_desc_init_bhsd_strides():
    d = abi.attn_desc_bhsd(2, 32, 67, 4374)
    assert (d.B, d.H, d.Sq, d.Sk, d.D) == (2, 32, 67, 4374, 64)
    assert list(d.q_stride) == [32 * 67 * 64, 67 * 64, 64]
    assert list(d.k_stride) == [32 * 4374 * 64, 4374 * 64, 64]
    assert list(d.o_stride) == list(d.q_stride)
    assert d.scale == 0.0 and d.num_splits == 0 and not d.kv_valid_len


def test_rejects_unsupported_before_launch():
    d = abi.attn_desc_bhsd(1, 2, 67, 67, D=128)
    assert _fwd(d) == abi.SF_ENOTSUP
    d = abi.attn_desc_bhsd(1, 2, 67, 67, in_dtype=abi.SF_I8)
    assert _fwd(d) == abi.SF_ENOTSUP
    d = abi.attn_desc_bhsd(1, 2, 67, 67, out_dtype=abi.SF_I8)
    assert _fwd(d) == abi.SF_ENOTSUP


def test_rejects_bad_arguments_before_launch():
    d = abi.attn_desc_bhsd(1, 2, 67, 67)
    assert abi.lib().sf_attn_fwd(None, 16, 16, 16, 16, None, 0, None) == abi.SF_EINVAL
    assert _fwd(d, q=None) == abi.SF_EINVAL
    assert _fwd(d, k=24) == abi.SF_EINVAL          # not 16-byte aligned
    d.q_stride[2] = 65                               # row stride not a multiple of 8
    assert _fwd(d) == abi.SF_EINVAL
    d = abi.attn_desc_bhsd(1, 2, 67, 0)
    assert _fwd(d) == abi.SF_EINVAL                 # keys required
    d = abi.attn_desc_bhsd(1, 2, 67, 67)
    d.num_splits = -1
    assert _fwd(d) == abi.SF_EINVAL
    # the output strides follow the same rules as the inputs
    d = abi.attn_desc_bhsd(1, 2, 67, 67)
    d.o_stride[2] = 68
    assert _fwd(d) == abi.SF_EINVAL
    d = abi.attn_desc_bhsd(1, 2, 67, 67)
    d.o_stride[1] = 4
    assert _fwd(d) == abi.SF_EINVAL
    # rows closer than D apart (a zero s-stride would give an empty buffer range)
    for name in ("q_stride", "k_stride", "v_stride", "o_stride"):
        for bad in (0, 56):
            d = abi.attn_desc_bhsd(1, 2, 67, 4374)
            getattr(d, name)[2] = bad
            assert _fwd(d) == abi.SF_EINVAL, (name, bad)


def test_gemm_single_pass_rejects_weights_beyond_32bit_range():
    """The workspace-free path addresses the whole weight through one 32-bit
    buffer range: a weight over 2 GiB is SF_ENOTSUP, not rows read as zeros."""
    g = abi.GemmDesc()
    g.M, g.N, g.K = 67, 1 << 20, 2048
    g.A, g.lda, g.a_dtype = 256, 2048, abi.SF_BF16
    g.W, g.ldw, g.w_dtype = 256, 2048, abi.SF_BF16
    g.epilogue, g.C, g.ldc, g.c_dtype = abi.SF_EPI_PLAIN, 256, 1 << 20, abi.SF_F32
    assert abi.lib().sf_gemm(ctypes.byref(g), None) == abi.SF_ENOTSUP
    g.w_dtype = abi.SF_I8                  # int8: 1 byte per weight, 2^31 + 2^20 bytes
    g.w_scale = 256
    g.N = (1 << 20) + 512
    g.ldc = g.N
    assert abi.lib().sf_gemm(ctypes.byref(g), None) == abi.SF_ENOTSUP


def _int8_direct(**over):
    g = abi.GemmDesc()
    g.M, g.N, g.K = 2144, 2048, 2048
    g.lda, g.a_dtype, g.ldw, g.w_dtype = 2048, abi.SF_F16, 2048, abi.SF_I8
    g.epilogue, g.c_dtype, g.act = abi.SF_EPI_PLAIN, abi.SF_F16, abi.SF_ACT_NONE
    for k, v in over.items():
        setattr(g, k, v)
    return abi.lib().sf_gemm_int8_direct(ctypes.byref(g))


def test_gemm_int8_direct_routing():
    """Which int8 calls above 160 rows sf_gemm multiplies directly (no
    16-bit copy of the codes): K = 2048, N % 256 == 0, ldw % 16 == 0, fp16
    activations, act NONE or GELU, an fp16 C or a round_product epilogue.
    Host logic only (no pointer is inspected)."""
    assert _int8_direct() == 1
    assert _int8_direct(act=abi.SF_ACT_GELU_TANH) == 1
    assert _int8_direct(M=161, N=256) == 1
    assert _int8_direct(N=6144) == 1
    assert _int8_direct(epilogue=abi.SF_EPI_ADD_NORM, c_dtype=abi.SF_F32, round_product=1) == 1
    assert _int8_direct(epilogue=abi.SF_EPI_HEADS, round_product=1) == 1
    assert _int8_direct(M=160) == 0                                   # the split-K regime
    assert _int8_direct(K=1024) == 0
    assert _int8_direct(N=2000) == 0
    assert _int8_direct(ldw=2056) == 0                                # rows not 16-byte aligned
    assert _int8_direct(w_codes16=256) == 0                           # a copy given: hipBLASLt on it
    assert _int8_direct(w_dtype=abi.SF_BF16) == 0
    assert _int8_direct(a_dtype=abi.SF_BF16, c_dtype=abi.SF_BF16) == 0
    assert _int8_direct(c_dtype=abi.SF_BF16) == 0
    assert _int8_direct(c_dtype=abi.SF_F32) == 0
    assert _int8_direct(accumulate=1) == 0
    assert _int8_direct(act=abi.SF_ACT_SILU) == 0
    assert _int8_direct(epilogue=abi.SF_EPI_ADD_NORM, c_dtype=abi.SF_F32) == 0   # fp32 product wanted
    assert abi.lib().sf_gemm_int8_direct(None) == 0


def test_empty_problem_is_a_noop():
    d = abi.attn_desc_bhsd(0, 32, 67, 4374)
    assert _fwd(d, None, None, None, None) == abi.SF_OK
    d = abi.attn_desc_bhsd(1, 32, 0, 4374)
    assert _fwd(d, None, None, None, None) == abi.SF_OK


def test_workspace_contract():
    d = abi.attn_desc_bhsd(1, 32, 67, 4374)
    ns = abi.lib().sf_attn_num_splits(ctypes.byref(d))
    assert ns > 1
    need = abi.lib().sf_attn_workspace_bytes(ctypes.byref(d))
    assert need == 1 * 32 * ns * 67 * (64 + 2) * 4
    assert _fwd(d, ws=None, wsn=0) == abi.SF_EWORKSPACE
    assert _fwd(d, ws=16, wsn=need - 4) == abi.SF_EWORKSPACE
    # self-attention needs no split, hence no workspace
    d1 = abi.attn_desc_bhsd(1, 32, 67, 67)
    assert abi.lib().sf_attn_num_splits(ctypes.byref(d1)) == 1
    assert abi.lib().sf_attn_workspace_bytes(ctypes.byref(d1)) == 0
    d1.num_splits = 3
    assert abi.lib().sf_attn_workspace_bytes(ctypes.byref(d1)) == 32 * 3 * 67 * 66 * 4
    d1.num_splits = 0
    d1.scale = -1.0
    assert _fwd(d1) == abi.SF_ENOTSUP


def test_query_block_calls_need_no_workspace():
    """Calls whose 80-row grid leaves CUs idle and whose keys fit 1024 run
    one workgroup per query block without a key split: split count 1, no
    workspace.  Longer key sets and grids that fill the CUs keep their
    split choice; a forced split count is honoured."""
    lib = abi.lib()
    for B, H, Sk in ((1, 32, 1024), (1, 32, 129), (2, 32, 700), (4, 32, 1024), (1, 3, 600)):
        d = abi.attn_desc_bhsd(B, H, 67, Sk)
        assert lib.sf_attn_num_splits(ctypes.byref(d)) == 1, (B, H, Sk)
        assert lib.sf_attn_workspace_bytes(ctypes.byref(d)) == 0, (B, H, Sk)
    assert lib.sf_attn_num_splits(ctypes.byref(abi.attn_desc_bhsd(1, 32, 67, 1025))) > 1
    assert lib.sf_attn_num_splits(ctypes.byref(abi.attn_desc_bhsd(1, 32, 67, 4374))) == 7
    d = abi.attn_desc_bhsd(1, 32, 67, 1024)
    d.num_splits = 2
    assert lib.sf_attn_workspace_bytes(ctypes.byref(d)) == 32 * 2 * 67 * 66 * 4


def test_backend_library_loads_and_exports_the_operator():
    """libsf_backend.so (the C++ RocmBackend over the C-ABI) loads on the host
    and exports RocmBackend::attention."""
    import ctypes
    import os
    import subprocess
    path = os.path.join(os.path.dirname(abi.LIB_PATH), "libsf_backend.so")
    abi.lib()
    ctypes.CDLL(path)
    syms = subprocess.run(["nm", "-DC", path], capture_output=True, text=True).stdout
    assert "sf_amd::RocmBackend::attention(" in syms
    assert "sf_amd::RocmBackend::reserve_attention_workspace(" in syms


def test_noalloc_rejects_before_touching_the_device():
    """sf_attn_fwd_noalloc validates and sizes its partials on the host: a bad
    descriptor and partials beyond the fixed scratch return without a HIP call."""
    d = abi.attn_desc_bhsd(1, 32, 67, 4374)
    d.D = 128
    assert abi.lib().sf_attn_fwd_noalloc(ctypes.byref(d), 16, 16, 16, 16, None) == abi.SF_ENOTSUP
    d = abi.attn_desc_bhsd(4, 32, 67, 4374)
    d.num_splits = 32
    assert abi.lib().sf_attn_workspace_bytes(ctypes.byref(d)) > abi.SF_ATTN_NOALLOC_SCRATCH_BYTES
    assert abi.lib().sf_attn_fwd_noalloc(ctypes.byref(d), 16, 16, 16, 16, None) == abi.SF_ESCRATCH


def test_auto_split_partials_fit_the_noalloc_scratch():
    """Every automatically chosen split count keeps its partials inside the
    allocation-free entry point's scratch."""
    worst = 0
    for B in (1, 2, 3, 4, 5, 8, 16):
        for H in (1, 8, 32):
            for Sq in (1, 16, 67, 80, 81, 160, 200, 1000):
                for Sk in (129, 1024, 4374, 65536, 1 << 20):
                    d = abi.attn_desc_bhsd(B, H, Sq, Sk)
                    worst = max(worst, abi.lib().sf_attn_workspace_bytes(ctypes.byref(d)))
    assert 0 < worst <= abi.SF_ATTN_NOALLOC_SCRATCH_BYTES


def test_int8_codes_to_bf16_rejects_bad_jobs():
    """Argument checks of the batched code widening, before any launch:
    too many jobs, K or the row stride not a multiple of 16, misaligned
    pointers, stride below K."""
    lib = abi.lib()
    jobs = (abi.CodesJob * (abi.SF_CODES_MAX_JOBS + 1))()
    for j in jobs:
        j.q, j.ldq, j.out, j.N, j.K = 256, 64, 512, 4, 64
    assert lib.sf_int8_codes_to_bf16(jobs, 0, None) == abi.SF_OK
    assert lib.sf_int8_codes_to_bf16(jobs, abi.SF_CODES_MAX_JOBS + 1, None) == abi.SF_EINVAL
    assert lib.sf_int8_codes_to_bf16(jobs, -1, None) == abi.SF_EINVAL
    for field, bad in (("K", 40), ("ldq", 72), ("ldq", 48), ("q", 264), ("out", 520), ("N", -1)):
        one = (abi.CodesJob * 1)()
        one[0].q, one[0].ldq, one[0].out, one[0].N, one[0].K = 256, 64, 512, 4, 64
        setattr(one[0], field, bad)
        assert lib.sf_int8_codes_to_bf16(one, 1, None) == abi.SF_EINVAL, (field, bad)


def test_weights_to_f16_rejects_bad_jobs():
    """Argument checks of the fp16 weight copies, before any launch: too
    many jobs, a source type other than int8 / bf16, K or the row stride
    (in bytes) not a multiple of 16, misaligned pointers, stride below K."""
    lib = abi.lib()
    jobs = (abi.W16Job * (abi.SF_CODES_MAX_JOBS + 1))()
    for j in jobs:
        j.w, j.w_dtype, j.ldw, j.out, j.N, j.K = 256, abi.SF_BF16, 64, 512, 4, 64
    assert lib.sf_weights_to_f16(jobs, 0, None) == abi.SF_OK
    assert lib.sf_weights_to_f16(jobs, abi.SF_CODES_MAX_JOBS + 1, None) == abi.SF_EINVAL
    assert lib.sf_weights_to_f16(jobs, -1, None) == abi.SF_EINVAL
    cases = [("K", 40, abi.SF_BF16), ("ldw", 48, abi.SF_BF16), ("w", 264, abi.SF_BF16), ("out", 520, abi.SF_BF16),
             ("N", -1, abi.SF_BF16), ("w_dtype", abi.SF_F32, abi.SF_F32), ("w_dtype", abi.SF_F16, abi.SF_F16),
             ("ldw", 72, abi.SF_I8), ("ldw", 68, abi.SF_BF16)]
    for field, bad, wd in cases:
        one = (abi.W16Job * 1)()
        one[0].w, one[0].w_dtype, one[0].ldw, one[0].out, one[0].N, one[0].K = 256, wd, 64, 512, 4, 64
        setattr(one[0], field, bad)
        assert lib.sf_weights_to_f16(one, 1, None) == abi.SF_EINVAL, (field, bad)


def test_absmax_batched_rejects_bad_jobs():
    """Argument checks of the batched max-|x| scan, before any launch: job
    count outside 0..SF_ABSMAX_MAX_JOBS, a missing output, a negative
    length, a misaligned buffer."""
    lib = abi.lib()
    jobs = (abi.AbsmaxJob * (abi.SF_ABSMAX_MAX_JOBS + 1))()
    for j in jobs:
        j.p, j.n, j.out = 256, 64, 512
    assert lib.sf_absmax_bf16_batched(jobs, 0, None) == abi.SF_OK
    assert lib.sf_absmax_bf16_batched(jobs, abi.SF_ABSMAX_MAX_JOBS + 1, None) == abi.SF_EINVAL
    assert lib.sf_absmax_bf16_batched(jobs, -1, None) == abi.SF_EINVAL
    for field, bad in (("out", None), ("n", -1), ("p", 264), ("p", None)):
        one = (abi.AbsmaxJob * 1)()
        one[0].p, one[0].n, one[0].out = 256, 64, 512
        setattr(one[0], field, bad)
        assert lib.sf_absmax_bf16_batched(one, 1, None) == abi.SF_EINVAL, (field, bad)


def test_gemm_partials_mode_contract():
    """sf_gemm_num_splits: the split-K slice count of a shape (0 above 160
    rows); SF_EPI_PARTIALS needs a call that runs split-K with a workspace
    (SF_ENOTSUP otherwise, before any launch)."""
    lib = abi.lib()
    g = abi.GemmDesc()
    g.M, g.N, g.K = 67, 2048, 2048
    g.A, g.lda, g.a_dtype = 256, 2048, abi.SF_BF16
    g.W, g.ldw, g.w_dtype = 512, 2048, abi.SF_BF16
    g.epilogue = abi.SF_EPI_PARTIALS
    assert lib.sf_gemm_num_splits(ctypes.byref(g)) == 8
    g.K = 8192   # 32 slices of 256 would exceed 16: 512-wide slices
    assert lib.sf_gemm_num_splits(ctypes.byref(g)) == 16
    g.K = 2048
    assert lib.sf_gemm(ctypes.byref(g), None) == abi.SF_ENOTSUP          # no workspace
    g.M = 161
    assert lib.sf_gemm_num_splits(ctypes.byref(g)) == 0
    g.workspace, g.workspace_bytes = 1024, 1 << 30
    assert lib.sf_gemm(ctypes.byref(g), None) == abi.SF_ENOTSUP          # library path


def test_ctypes_mirrors_match_the_c_layout(tmp_path):
    """Every ctypes mirror of an include/*.h struct has the C compiler's size
    and field offsets (a field added to a header but not to its mirror would
    shift every later field the Python front ends write)."""
    import shutil
    import subprocess

    from servoflow_amd import rdt

    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    mirrors = {"sf_attn_desc": abi.AttnDesc, "sf_gemm_desc": abi.GemmDesc, "sf_codes_job": abi.CodesJob, "sf_w16_job": abi.W16Job,
               "sf_absmax_job": abi.AbsmaxJob, "sf_rdt_config": rdt.RdtConfig, "sf_st_entry": rdt.StEntry}
    lines = ['#include <stdio.h>', '#include "sf_rdt.h"', 'int main(void) {']
    for cname, py in mirrors.items():
        lines.append(f'  printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, *_ in py._fields_:
            lines.append(f'  printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines += ['  return 0;', '}']
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run([cc, "-std=c11", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = {}
    for line in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines():
        cname, field, val = line.split()
        got[(cname, field)] = int(val)
    for cname, py in mirrors.items():
        assert got[(cname, "size")] == ctypes.sizeof(py), cname
        for fname, *_ in py._fields_:
            assert got[(cname, fname)] == getattr(py, fname).offset, (cname, fname)


def test_qk_norm_on_load_contract():
    """q_gamma / k_gamma without q_partials: bf16 inputs only, 16-byte
    aligned weights, K normalised only on the short-key (Sk <= 128) path."""
    d = abi.attn_desc_bhsd(1, 2, 67, 67)
    d.q_gamma = 24
    assert _fwd(d) == abi.SF_EINVAL
    d.q_gamma, d.k_gamma = 16, 40
    assert _fwd(d) == abi.SF_EINVAL
    d = abi.attn_desc_bhsd(1, 2, 67, 67, in_dtype=abi.SF_F16)
    d.q_gamma = 24
    assert _fwd(d) == abi.SF_EINVAL   # fp16 rows take the norm too (alignment still checked)
    d = abi.attn_desc_bhsd(1, 2, 67, 67, in_dtype=abi.SF_F32)
    d.q_gamma = 16
    assert _fwd(d) == abi.SF_ENOTSUP
    d = abi.attn_desc_bhsd(1, 2, 67, 67, in_dtype=abi.SF_F32)
    d.k_gamma = 16
    assert _fwd(d) == abi.SF_ENOTSUP
    d = abi.attn_desc_bhsd(1, 2, 67, 4374)
    d.k_gamma = 16
    assert _fwd(d) == abi.SF_ENOTSUP
    d = abi.attn_desc_bhsd(1, 2, 67, 67)
    d.num_splits, d.k_gamma = 2, 16
    assert _fwd(d) == abi.SF_ENOTSUP


def test_q_f16_contract():
    """q_f16 (fp16 Q rows against bf16 K / V): bf16 in_dtype only, and not
    with Q given as projection partials."""
    for dt in (abi.SF_F16, abi.SF_F32):
        d = abi.attn_desc_bhsd(1, 2, 67, 4374, in_dtype=dt)
        d.q_f16 = 1
        assert _fwd(d) == abi.SF_ENOTSUP, dt
    d = abi.attn_desc_bhsd(1, 2, 67, 512)
    d.q_f16, d.q_partials, d.q_splits = 1, 256, 2
    assert _fwd(d) == abi.SF_ENOTSUP


def test_gemm_algo_timing_switch_arguments():
    lib = abi.lib()
    for bad in (-1, 2, 7):
        assert lib.sf_gemm_set_algo_timing(bad) == abi.SF_EINVAL
    assert lib.sf_gemm_set_algo_timing(1) == abi.SF_OK   # the default, restored
