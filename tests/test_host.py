"""Host-side checks that need no GPU: the C ABI library loads and exports every declared
entry point, the ctypes struct mirror matches the C layout, and the Python interface keeps
the reference's argument checking and error behaviour."""

import ctypes
import os
import re
import subprocess
import tempfile

import pytest
import torch

import fa4_ring
from fa4_ring import _lib
from fa4_ring.config import RingConfig
from fa4_ring.fa4_backend import _norm_descale, fa4_attn, sweep_descales
from fa4_ring.merge import BatchedMerger, IncrementalMerger, make_merger
from fa4_ring.ring_attention import Descales, LocalKVRing, ring_flash_attn
from fa4_ring.zigzag import get_half_index, half_indices, local_seqlen

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fa4cp.h")


def _declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(fa4cp_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    syms = _declared_symbols()
    assert len(syms) >= 7
    for s in syms:
        assert hasattr(lib, s), f"{s} declared in include/fa4cp.h but not exported"
    assert set(syms) <= set(_lib.SIGNATURES), "every declared entry point has a ctypes signature"
    assert lib.fa4cp_abi_version() == _lib.ABI_VERSION


def test_error_path_reports_message_without_gpu():
    lib = _lib.load()
    # invalid arguments are rejected before any HIP call
    rc = lib.fa4cp_merge_states(None, None, None, None, 1, 1, 1, 8, 0, None)
    assert rc == -1
    assert b"null pointer" in lib.fa4cp_last_error()
    rc = lib.fa4cp_zigzag_shard(1, 1, 16, None, 1, 10, 0, 4, None)
    assert rc == -1 and b"divisible" in lib.fa4cp_last_error()
    # the merges read 16-byte vectors of v: misaligned tensors are refused
    rc = lib.fa4cp_merge_states(1 << 20 | 8, 1 << 20, 1 << 21, 1 << 21, 4, 2, 8, 128, 0, None)
    assert rc == -1 and b"aligned" in lib.fa4cp_last_error()
    rc = lib.fa4cp_merge_state_inplace(1 << 20, 1 << 20, 1 << 21 | 2, 1 << 21, 4, 8, 128, 0, None, 0, 0, None)
    assert rc == -1 and b"aligned" in lib.fa4cp_last_error()
    a = _lib.AttnArgs()
    a.total_q = 1
    rc = lib.fa4cp_attn_fwd(ctypes.byref(a), None)
    assert rc == -1 and b"null tensor" in lib.fa4cp_last_error()
    with pytest.raises(RuntimeError, match="null tensor"):
        _lib.check(rc, "fa4cp_attn_fwd")


def test_empty_calls_launch_nothing_and_take_null_pointers():
    """A call with no rows returns 0 before any HIP call, whatever the pointers of its empty
    tensors (torch gives NULL for zero-element tensors); with rows, NULL is still an error."""
    lib = _lib.load()
    bf16 = _lib.dtype_code(torch.bfloat16)
    a = _lib.AttnArgs()
    a.q_row_stride, a.q_head_stride = 8 * 128, 128
    a.k_row_stride, a.k_head_stride = 2 * 128, 128
    a.v_row_stride, a.v_head_stride = 2 * 128, 128
    a.o_row_stride, a.o_head_stride = 8 * 128, 128
    a.lse_row_stride = 8
    a.h_q, a.h_kv, a.d, a.dtype, a.causal = 8, 2, 128, bf16, 1
    assert lib.fa4cp_attn_fwd(ctypes.byref(a), None) == 0
    a.total_q = a.total_k = 64
    assert lib.fa4cp_attn_fwd(ctypes.byref(a), None) == -1 and b"null" in lib.fa4cp_last_error()

    s = _lib.SweepArgs()
    s.q_row_stride, s.q_head_stride = 8 * 128, 128
    s.o_row_stride, s.o_head_stride = 8 * 128, 128
    s.lse_row_stride = 8
    s.k_row_stride, s.k_head_stride = 2 * 128, 128
    s.vt_d_stride = int(lib.fa4cp_vt_min_d_stride(0, 1))
    s.h_q, s.h_kv, s.d, s.dtype = 8, 2, 128, bf16
    s.cp_rank, s.cp_size, s.softmax_scale = 1, 4, 0.1
    assert lib.fa4cp_ring_sweep_fwd(ctypes.byref(s), None) == 0
    s.total = 64
    assert lib.fa4cp_ring_sweep_fwd(ctypes.byref(s), None) == -1 and b"null" in lib.fa4cp_last_error()

    for rows, want in ((0, 0), (4, -1)):
        assert lib.fa4cp_merge_state_inplace(None, None, None, None, rows, 8, 128, bf16, None, 0, 0, None) == want
        assert lib.fa4cp_merge_states(None, None, None, None, rows, 2, 8, 128, bf16, None) == want
    for n, want in ((0, 0), (64, -1)):
        assert lib.fa4cp_zigzag_shard(None, None, 256, None, 1, n, 0, 4, None) == want
        assert lib.fa4cp_zigzag_unshard((ctypes.c_void_p * 4)(), None, 256, None, 1, n, 4, None) == want


def test_paged_entry_points_validate_before_launching():
    """fa4cp_gather_kv_pages / fa4cp_transpose_v_paged_many: nothing to do returns 0, bad
    page geometry, strides, counts and types are rejected, all before any HIP call."""
    lib = _lib.load()

    def args(**kw):
        a = _lib.PagedArgs()
        a.total, a.h_kv, a.d, a.dtype = 0, 2, 128, _lib.dtype_code(torch.bfloat16)
        a.page_size, a.num_pages, a.pt_stride = 128, 4, 1
        a.cache_row_stride, a.cache_head_stride = 256, 128
        for key, val in kw.items():
            setattr(a, key, val)
        return a

    arr = (ctypes.c_void_p * 1)()
    assert lib.fa4cp_gather_kv_pages(ctypes.byref(args()), arr, arr, arr, 256, 128, 1, None) == 0
    assert lib.fa4cp_transpose_v_paged_many(ctypes.byref(args()), arr, arr, arr, 128, 1, None) == 0
    cases = [(dict(page_size=96), b"page_size"), (dict(page_size=0), b"page_size"),
             (dict(total=1000, pt_stride=7), b"pt_stride"), (dict(cache_row_stride=100), b"16-byte"),
             (dict(dtype=9), b"dtype"), (dict(h_kv=0), b"bad shape")]
    for kw, msg in cases:
        for rc in (lib.fa4cp_gather_kv_pages(ctypes.byref(args(**kw)), arr, arr, arr, 256, 128, 1, None),
                   lib.fa4cp_transpose_v_paged_many(ctypes.byref(args(**kw)), arr, arr, arr, 1024, 1, None)):
            assert rc != 0 and msg in lib.fa4cp_last_error(), (kw, lib.fa4cp_last_error())
    rc = lib.fa4cp_gather_kv_pages(ctypes.byref(args()), arr, arr, arr, 256, 128, 0, None)
    assert rc != 0 and b"count" in lib.fa4cp_last_error()
    rc = lib.fa4cp_gather_kv_pages(ctypes.byref(args(total=256, pt_stride=2)), arr, arr, arr, 256, 128, 1, None)
    assert rc != 0 and b"null" in lib.fa4cp_last_error()


def test_paged_ring_checks_its_caches():
    """PagedKVRing refuses caches that are not [num_pages, page_size, H_kv, D], host tensors
    and mismatched lists before anything reaches the library."""
    from fa4_ring import PagedKVRing

    c = torch.zeros(4, 128, 2, 64, dtype=torch.bfloat16)
    pt = torch.zeros(1, 4, dtype=torch.int32)
    with pytest.raises(AssertionError, match="num_pages, page_size"):
        PagedKVRing([c[0]], [c[0]], [pt])
    with pytest.raises(AssertionError, match="device tensors"):
        PagedKVRing([c], [c], [pt])
    with pytest.raises(AssertionError, match="per source rank"):
        PagedKVRing([c, c], [c], [pt, pt])


def test_sweep_entry_point_validates_before_launching():
    """fa4cp_ring_sweep_fwd rejects bad arguments with a message and no HIP call: null
    sources, cp_rank / cp_size out of range, a negative max_seqlen, unsupported head dims.
    The pointers are fake, so this never runs where a device is visible."""
    if torch.cuda.device_count() > 0:
        pytest.skip("fake device pointers: host-only test")
    lib = _lib.load()
    fake = 1 << 20  # never dereferenced: every case fails validation first

    def args(**kw):
        a = _lib.SweepArgs()
        a.q = a.out = a.lse = fake
        a.q_row_stride, a.q_head_stride = 8 * 128, 128
        a.o_row_stride, a.o_head_stride = 8 * 128, 128
        a.lse_row_stride = 8
        a.k_row_stride, a.k_head_stride = 2 * 128, 128
        a.vt_d_stride = int(lib.fa4cp_vt_min_d_stride(256, 1))
        a.total, a.h_q, a.h_kv, a.d = 256, 8, 2, 128
        a.dtype = _lib.dtype_code(torch.bfloat16)
        a.cp_rank, a.cp_size = 0, 2
        a.softmax_scale = 0.1
        for i in range(2):
            a.k[i] = a.v_t[i] = fake
        for key, val in kw.items():
            setattr(a, key, val)
        return a

    cases = [(dict(cp_size=0), b"out of range"), (dict(cp_rank=2), b"out of range"),
             (dict(cp_size=_lib.MAX_CP + 1), b"out of range"), (dict(cu=fake, nseq=1, max_seqlen=-4), b"max_seqlen"),
             (dict(d=96), b"head dim"), (dict(h_q=7), b"multiple")]
    for kw, msg in cases:
        a = args(**kw)
        rc = lib.fa4cp_ring_sweep_fwd(ctypes.byref(a), None)
        assert rc != 0 and msg in lib.fa4cp_last_error(), (kw, lib.fa4cp_last_error())
    a = args()
    a.k[1] = 0
    assert lib.fa4cp_ring_sweep_fwd(ctypes.byref(a), None) != 0 and b"source 1" in lib.fa4cp_last_error()

    # the paged-K form: the same checks, plus its page geometry and tables
    def kpages(**kw):
        kp = _lib.SweepKPages()
        kp.pt_stride, kp.page_size, kp.num_pages = 2, 128, 4
        for i in range(2):
            kp.page_table[i] = fake
        for key, val in kw.items():
            setattr(kp, key, val)
        return kp

    assert lib.fa4cp_ring_sweep_fwd_paged(ctypes.byref(args()), None, None) != 0
    assert b"null k_pages" in lib.fa4cp_last_error()
    for kw, msg in [(dict(page_size=96), b"page_size"), (dict(page_size=0), b"page_size"),
                    (dict(num_pages=-1), b"num_pages"), (dict(pt_stride=1), b"pt_stride"),
                    (dict(pt_stride=1 << 31), b"pt_stride")]:
        rc = lib.fa4cp_ring_sweep_fwd_paged(ctypes.byref(args()), ctypes.byref(kpages(**kw)), None)
        assert rc != 0 and msg in lib.fa4cp_last_error(), (kw, lib.fa4cp_last_error())
    kp = kpages()
    kp.page_table[1] = 0
    rc = lib.fa4cp_ring_sweep_fwd_paged(ctypes.byref(args()), ctypes.byref(kp), None)
    assert rc != 0 and b"page table of source 1" in lib.fa4cp_last_error()
    rc = lib.fa4cp_ring_sweep_fwd_paged(ctypes.byref(args(cp_rank=3)), ctypes.byref(kpages()), None)
    assert rc != 0 and b"out of range" in lib.fa4cp_last_error()
    kp = kpages()
    kp.page_table[0] = kp.page_table[1] = 0
    assert lib.fa4cp_ring_sweep_fwd_paged(ctypes.byref(args(total=0)), ctypes.byref(kp), None) == 0


def test_backward_workspace_size_and_checks():
    """fa4cp_ring_sweep_bwd_workspace_bytes: delta (total x h_q float32, rounded up to 256
    bytes) plus h_q x (padded rows / 32) packed blocks of 4 x 64 x d + 256 bytes each, and
    cp_size x h_kv x (padded rows / 32) K / V blocks of 3 x 64 x d bytes; the
    backward refuses a workspace that is small or not 256-byte aligned before any HIP call.
    The pointers are fake, so this never runs where a device is visible."""
    if torch.cuda.device_count() > 0:
        pytest.skip("fake device pointers: host-only test")
    lib = _lib.load()
    fake = 1 << 20

    def args(**kw):
        a = _lib.SweepBwdArgs()
        a.q = a.dout = a.out = a.lse = a.dq = a.workspace = fake
        a.q_row_stride = a.do_row_stride = a.o_row_stride = 8 * 128
        a.q_head_stride = a.do_head_stride = a.o_head_stride = 128
        a.lse_row_stride = 8
        a.k_row_stride = a.v_row_stride = 2 * 128
        a.k_head_stride = a.v_head_stride = 128
        a.total, a.h_q, a.h_kv, a.d = 256, 8, 2, 128
        a.dtype = _lib.dtype_code(torch.bfloat16)
        a.cp_rank, a.cp_size = 0, 2
        a.softmax_scale = 0.1
        for i in range(2):
            a.k[i] = a.v[i] = a.dk[i] = a.dv[i] = fake
        for key, val in kw.items():
            setattr(a, key, val)
        return a

    def expect(total, nseq, h_q, d):
        delta = -(-total * h_q * 4 // 256) * 256
        # rows of the padded layout: every sequence padded to a multiple of 128 rows fits in
        # total + 128 nseq, rounded up to 128 (fa4cp_vt_min_d_stride)
        rows = -(-(total + 128 * nseq) // 128) * 128
        assert rows == lib.fa4cp_vt_min_d_stride(total, nseq)
        kv = 2 * 2 * (rows // 32) * 3 * 64 * d  # K / V blocks (cp 2, h_kv 2)
        return delta + h_q * (rows // 32) * (4 * 64 * d + 256) + kv

    # one sequence of 256 rows: 384 padded rows, so 8 heads x 12 blocks of 33024 bytes + 8 KB, and
    # 2 sources x 2 kv heads x 12 key blocks of 24576 bytes
    assert lib.fa4cp_ring_sweep_bwd_workspace_bytes(ctypes.byref(args())) == 8192 + 8 * 12 * 33024 + 4 * 12 * 24576
    for total, nseq, h_q, d in [(256, 1, 8, 128), (100, 1, 3, 64), (16384, 1, 32, 128), (1000, 7, 4, 64),
                                (512, 1, 4, 256)]:
        a = args(total=total, h_q=h_q, d=d, nseq=nseq, cu=fake if nseq > 1 else None)
        assert lib.fa4cp_ring_sweep_bwd_workspace_bytes(ctypes.byref(a)) == expect(total, nseq, h_q, d)
    for kw, msg in [(dict(d=96), b"bad shape"), (dict(h_q=0), b"bad shape"), (dict(total=-1), b"bad shape"),
                    (dict(cu=fake, nseq=0), b"bad shape")]:
        assert lib.fa4cp_ring_sweep_bwd_workspace_bytes(ctypes.byref(args(**kw))) < 0
        assert msg in lib.fa4cp_last_error(), kw
    assert lib.fa4cp_ring_sweep_bwd_workspace_bytes(None) < 0

    need = lib.fa4cp_ring_sweep_bwd_workspace_bytes(ctypes.byref(args()))
    for kw, msg in [(dict(workspace_bytes=need - 1), b"workspace"), (dict(workspace_bytes=need, workspace=fake + 16),
                                                                     b"workspace"),
                    (dict(workspace=None, workspace_bytes=need), b"workspace"), (dict(d=96), b"head dim"),
                    (dict(cp_rank=2), b"cp_rank")]:
        rc = lib.fa4cp_ring_sweep_bwd(ctypes.byref(args(**kw)), None)
        assert rc != 0 and msg in lib.fa4cp_last_error(), (kw, lib.fa4cp_last_error())
    # nothing to do: no workspace needed
    assert lib.fa4cp_ring_sweep_bwd(ctypes.byref(args(total=0, workspace=None)), None) == 0


@pytest.mark.parametrize("struct,cname", [(_lib.AttnArgs, "fa4cp_attn_args"),
                                           (_lib.TransposeArgs, "fa4cp_transpose_args"),
                                           (_lib.SweepArgs, "fa4cp_sweep_args"),
                                           (_lib.SweepBwdArgs, "fa4cp_sweep_bwd_args"),
                                           (_lib.QuantArgs, "fa4cp_quant_args"),
                                           (_lib.PagedArgs, "fa4cp_paged_args"),
                                           (_lib.SweepKPages, "fa4cp_sweep_kpages")])
def test_args_layout_matches_c_header(struct, cname):
    fields = [f for f, _ in struct._fields_]
    prog = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"', "int main(void){",
            f'printf("%zu\\n", sizeof({cname}));']
    prog += [f'printf("%zu\\n", offsetof({cname}, {f}));' for f in fields]
    prog.append("return 0;}")
    with tempfile.TemporaryDirectory() as td:
        src, exe = os.path.join(td, "l.c"), os.path.join(td, "l")
        open(src, "w").write("\n".join(prog))
        subprocess.run(["gcc", "-o", exe, src], check=True)
        vals = [int(x) for x in subprocess.run([exe], check=True, capture_output=True,
                                               text=True).stdout.split()]
    assert vals[0] == ctypes.sizeof(struct)
    for f, off in zip(fields, vals[1:]):
        assert getattr(struct, f).offset == off, f


def test_ring_config_checks():
    RingConfig(cp_size=8, cp_rank=7)
    with pytest.raises(AssertionError):
        RingConfig(cp_size=4, cp_rank=4)
    with pytest.raises(AssertionError):
        RingConfig(cp_size=0, cp_rank=0)
    with pytest.raises(AssertionError):
        RingConfig(cp_size=2, cp_rank=0, causal=False)
    with pytest.raises(AssertionError):
        RingConfig(cp_size=2, cp_rank=0, merge_mode="tree")


def test_make_merger():
    assert isinstance(make_merger("incremental"), IncrementalMerger)
    assert isinstance(make_merger("batched"), BatchedMerger)
    with pytest.raises(ValueError):
        make_merger("nope")
    with pytest.raises(AssertionError):
        IncrementalMerger().result()
    with pytest.raises(AssertionError):
        BatchedMerger().result()
    # one partial is returned as is
    b = BatchedMerger()
    t = torch.zeros(2, 1, 8)
    b.add(t, torch.zeros(2, 1))
    assert b.result() is t


def test_sweep_descales_one_table():
    """The fused sweep's q / k / v descales come back as rows of one stack, each equal to the
    per-part normalisation, contiguous, float32; a part given as None comes back None."""
    ks = [torch.tensor(0.5), torch.arange(4.0) + 1, torch.full((1, 4), 3.0)]
    vs = [torch.tensor(2.0, dtype=torch.float64), torch.tensor(4.0), torch.arange(4.0).reshape(1, 4)]
    q = torch.tensor(0.25)
    qd, kd, vd = sweep_descales(q, ks, vs, 4, "cpu")
    assert qd.tolist() == [0.25] * 4 and qd.is_contiguous() and qd.dtype == torch.float32
    assert kd.shape == (3, 4) and kd.is_contiguous() and vd.shape == (3, 4) and vd.is_contiguous()
    assert kd.tolist() == [_norm_descale(k, 4, "cpu").tolist() for k in ks]
    assert vd.tolist() == [_norm_descale(v, 4, "cpu").tolist() for v in vs]
    assert kd.dtype == vd.dtype == torch.float32
    qd, kd, vd = sweep_descales(None, ks, None, 4, "cpu")
    assert qd is None and vd is None and kd.tolist() == [_norm_descale(k, 4, "cpu").tolist() for k in ks]
    assert sweep_descales(None, None, None, 4, "cpu") == (None, None, None)
    qd, kd, vd = sweep_descales(q, None, vs[:1], 4, "cpu")
    assert kd is None and qd.tolist() == [0.25] * 4 and vd.tolist() == [[2.0] * 4]


def test_norm_descale_shapes():
    assert _norm_descale(None, 4, "cpu") is None
    assert _norm_descale(torch.tensor(0.5), 4, "cpu").tolist() == [0.5] * 4
    assert _norm_descale(torch.arange(4.0), 4, "cpu").tolist() == [0, 1, 2, 3]
    assert _norm_descale(torch.arange(4.0).reshape(1, 4), 4, "cpu").tolist() == [0, 1, 2, 3]
    assert _norm_descale(torch.tensor(2, dtype=torch.float64), 2, "cpu").dtype == torch.float32
    with pytest.raises(AssertionError):
        _norm_descale(torch.ones(3), 4, "cpu")


def test_index_helpers_kat():
    f, s = half_indices(8, torch.device("cpu"))
    assert f.tolist() == [0, 1, 2, 3] and s.tolist() == [4, 5, 6, 7]
    cu = torch.tensor([0, 4, 12], dtype=torch.int32)
    assert get_half_index(cu, front=True).tolist() == [0, 1, 4, 5, 6, 7]
    assert get_half_index(cu, front=False).tolist() == [2, 3, 8, 9, 10, 11]
    assert local_seqlen(64, 4) == 16
    with pytest.raises(AssertionError):
        local_seqlen(30, 4)


def test_device_entry_points_reject_host_tensors():
    q = torch.zeros(16, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(AssertionError, match="device tensor"):
        fa4_attn(q, q, q, causal=True)
    with pytest.raises(AssertionError, match="device tensor"):
        fa4_ring.zigzag_shard(q, 0, 2)


def test_ring_without_local_kv_source_raises():
    q = torch.zeros(16, 2, 128, dtype=torch.bfloat16)
    cfg = RingConfig(cp_size=2, cp_rank=0)
    with pytest.raises(RuntimeError, match="LocalKVRing"):
        ring_flash_attn(q, q, q, cfg)
    with pytest.raises(AssertionError):
        ring_flash_attn(q, q, q, cfg, cu_seqlens=torch.tensor([0, 16], dtype=torch.int32))
    ring = LocalKVRing([q, q, q], [q, q, q])
    with pytest.raises(AssertionError, match="3 shards"):
        ring_flash_attn(q, q, q, cfg, group=ring)


def test_fused_sweep_rejects_what_it_does_not_cover():
    """fused=True is refused (AssertionError, before any device work) outside the fused
    kernel's cases: fp32, cp_size 1 or above 16, bf16 with descales.  Head dims above 256
    are refused for every form."""
    cfg = RingConfig(cp_size=2, cp_rank=0)

    def ring_of(x):
        return LocalKVRing([x, x], [x, x])

    x = torch.zeros(16, 2, 128, dtype=torch.float32)
    with pytest.raises(AssertionError, match="fused ring sweep"):
        ring_flash_attn(x, x, x, cfg, group=ring_of(x), fused=True)
    for dt in (torch.bfloat16, torch.float8_e4m3fn):
        x = torch.zeros(16, 2, 320, dtype=dt)
        with pytest.raises(AssertionError, match="head dim 320"):
            ring_flash_attn(x, x, x, cfg, group=ring_of(x))
    x = torch.zeros(16, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(AssertionError, match="fused ring sweep"):
        ring_flash_attn(x, x, x, cfg, group=ring_of(x), fused=True, descales=Descales(q=torch.tensor(1.0)))
    with pytest.raises(AssertionError, match="fused ring sweep"):
        ring_flash_attn(x, x, x, RingConfig(cp_size=1, cp_rank=0), fused=True)
    big = RingConfig(cp_size=17, cp_rank=0)
    with pytest.raises(AssertionError, match="fused ring sweep"):
        ring_flash_attn(x, x, x, big, group=LocalKVRing([x] * 17, [x] * 17), fused=True)


def test_kernel_head_dim_and_padding():
    """Head dims without a kernel run at the next supported one on zero-padded copies."""
    from fa4_ring.fa4_backend import kernel_head_dim, pad_head_dim
    bf, e8 = torch.bfloat16, torch.float8_e4m3fn
    assert [kernel_head_dim(bf, d) for d in (1, 32, 64, 65, 96, 128, 129, 192, 256)] == \
        [64, 64, 64, 128, 128, 128, 256, 256, 256]
    assert [kernel_head_dim(e8, d) for d in (16, 64, 128, 160, 256)] == [128, 128, 128, 256, 256]
    for dt, d in ((bf, 257), (e8, 300), (bf, 0)):
        with pytest.raises(AssertionError, match="head dim"):
            kernel_head_dim(dt, d)
    with pytest.raises(AssertionError, match="dtype"):
        kernel_head_dim(torch.float32, 128)
    x = torch.randn(5, 3, 80).to(bf)
    y = pad_head_dim(x, 128)
    assert y.shape == (5, 3, 128) and y.is_contiguous() and torch.equal(y[..., :80], x)
    assert torch.all(y[..., 80:] == 0)
    assert pad_head_dim(x, 80) is x
    z = torch.randn(5, 80, 3).to(bf).transpose(1, 2)  # not contiguous in D
    assert pad_head_dim(z, 80).is_contiguous() and torch.equal(pad_head_dim(z, 80), z)
    q8 = torch.randn(4, 2, 64).to(e8)
    p8 = pad_head_dim(q8, 128)
    assert p8.dtype == e8 and torch.equal(p8[..., :64].view(torch.uint8), q8.view(torch.uint8))
    assert torch.all(p8[..., 64:].view(torch.uint8) == 0)


def test_descale_table_forms():
    """Per-source descales in every accepted form (Python float, scalar, [H_kv], (1, H_kv))
    become one contiguous float32 [S, H_kv] table; a wrong shape is refused."""
    from fa4_ring.fa4_backend import descale_table
    ds = [0.25, torch.tensor(0.5), torch.tensor([1.0, 2.0], dtype=torch.float64), torch.tensor([[3.0, 4.0]])]
    t = descale_table(ds, 2, torch.device("cpu"))
    assert t.dtype == torch.float32 and t.is_contiguous() and t.shape == (4, 2)
    assert t.tolist() == [[0.25, 0.25], [0.5, 0.5], [1.0, 2.0], [3.0, 4.0]]
    with pytest.raises(AssertionError, match="descale"):
        descale_table([torch.tensor([1.0, 2.0, 3.0])], 2, torch.device("cpu"))


def test_max_seqlen_below_the_longest_sequence_is_refused():
    """max_seqlen sizes the kernels' grids: a bound below the longest local sequence would
    leave rows unwritten, so it is refused before any device work."""
    cfg = RingConfig(cp_size=1, cp_rank=0)
    q = torch.zeros(16, 2, 128, dtype=torch.bfloat16)
    cu = torch.tensor([0, 6, 16], dtype=torch.int32)
    with pytest.raises(AssertionError, match="max_seqlen 8 is below the longest local sequence"):
        ring_flash_attn(q, q, q, cfg, cu_seqlens=cu, max_seqlen=8)


def test_odd_local_lengths_are_refused():
    """A local sequence is two zig-zag chunks of equal size: an odd length (one sequence, or
    any packed one) is refused with AssertionError before any device work, as the
    reference's get_half_index refuses it."""
    cfg = RingConfig(cp_size=1, cp_rank=0)
    q = torch.zeros(15, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(AssertionError, match="odd length"):
        ring_flash_attn(q, q, q, cfg)
    q = torch.zeros(16, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(AssertionError, match=r"sequences \[1, 2\] have odd length"):
        ring_flash_attn(q, q, q, cfg, cu_seqlens=torch.tensor([0, 6, 11, 16], dtype=torch.int32), max_seqlen=6)
    with pytest.raises(AssertionError, match="even length"):
        get_half_index(torch.tensor([0, 6, 11], dtype=torch.int32), front=True)


def test_kv_shards_not_contiguous_in_d_are_copied():
    """The sweep's arguments carry K's row and head strides only, so LocalKVRing keeps a
    contiguous copy of a K or V view whose head dim is strided (as the reference copies with
    .contiguous() before FA4); shards already contiguous in D are kept as given."""
    x = torch.randn(16, 128, 2).to(torch.bfloat16).transpose(1, 2)  # [16, 2, 128], stride(2) = 2
    ok = torch.zeros(16, 2, 128, dtype=torch.bfloat16)
    ring = LocalKVRing([ok, x], [ok, x])
    assert ring.k[0] is ok and ring.v[0] is ok
    for t in (ring.k[1], ring.v[1]):
        assert t.stride(2) == 1 and t.stride() == ok.stride() and torch.equal(t, x)


def test_merge_entry_points_validate_without_gpu():
    lib = _lib.load()
    ptrs = (ctypes.c_void_p * 2)(1 << 20, 1 << 21)
    for n in (0, 17):
        assert lib.fa4cp_merge_states_list(ptrs, ptrs, n, 1 << 22, 1 << 23, 4, 2, 64, 0, None) == -1
        assert b"num_states" in lib.fa4cp_last_error()
    bad = (ctypes.c_void_p * 2)(1 << 20, (1 << 21) | 4)
    assert lib.fa4cp_merge_states_list(bad, ptrs, 2, 1 << 22, 1 << 23, 4, 2, 64, 0, None) == -1
    assert b"aligned" in lib.fa4cp_last_error()
    assert lib.fa4cp_merge_states_list(ptrs, ptrs, 2, None, None, 4, 2, 64, 0, None) == -1
    assert b"null" in lib.fa4cp_last_error()
    assert lib.fa4cp_merge_state(1 << 20, 1 << 20, 1 << 21, 1 << 21, None, None, 4, 2, 64, 0, None, 0, 0,
                                 None) == -1
    assert b"null" in lib.fa4cp_last_error()
    assert lib.fa4cp_merge_state(1 << 20, 1 << 20, 1 << 21, 1 << 21, 1 << 22, 1 << 23, 3, 2, 64, 0, None, 0,
                                 2, None) == -1
    assert b"even" in lib.fa4cp_last_error()
    # nothing to merge: no launch, NULL accepted
    assert lib.fa4cp_merge_states_list(ptrs, ptrs, 2, None, None, 0, 2, 64, 0, None) == 0


def test_public_api_names():
    for name in ["RingConfig", "ring_flash_attn", "Descales", "zigzag_shard", "zigzag_unshard",
                 "IncrementalMerger", "BatchedMerger", "make_merger", "LocalKVRing", "quantize_e4m3",
                 "quantize_ring"]:
        assert hasattr(fa4_ring, name)
    from fa4_ring.zigzag import zigzag_shard_varlen  # noqa: F401
    from fa4_ring.reference import full_causal_reference  # noqa: F401
    from fa4_ring.fa4_backend import has_fa4

    assert has_fa4() is True
