"""C ABI of libmtlattn_hip.so without a GPU: the library loads, exports every
function include/mtlattn_capi.h declares, and its host-side validation,
routing and workspace arithmetic behave as documented. No kernel is launched
(every call here fails validation or only queries sizes)."""

import ctypes
import os
import re

import pytest
import torch  # noqa: F401  (loads the HIP runtime the library binds to)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mtlattn_capi.h")
LIB = os.path.join(ROOT, "mtlattn_amd", "libmtlattn_hip.so")

F32, F16, BF16 = 0, 1, 2
OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_WORKSPACE = 0, -1, -2, -3


class Problem(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("num_seqs", ctypes.c_int32),
        ("total_q", ctypes.c_int64), ("total_kv", ctypes.c_int64),
        ("num_heads_q", ctypes.c_int32), ("num_heads_kv", ctypes.c_int32),
        ("head_dim", ctypes.c_int32), ("max_seqlen_q", ctypes.c_int32),
        ("scale", ctypes.c_float), ("causal", ctypes.c_int32), ("window", ctypes.c_int32),
        ("cu_seqlens_q", ctypes.c_void_p), ("cu_seqlens_kv", ctypes.c_void_p),
        ("bias", ctypes.c_void_p), ("bias_q_stride", ctypes.c_int64),
        ("bias_h_stride", ctypes.c_int64), ("bias_kv_cols", ctypes.c_int64),
        ("bias_seq_local", ctypes.c_int32), ("bias_seq_stride", ctypes.c_int64),
        ("bias_seq_rows", ctypes.c_int64),
    ]


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail("libmtlattn_hip.so is not built (run __graft_entry__.build())")
    L = ctypes.CDLL(LIB)
    L.mtlattn_last_error.restype = ctypes.c_char_p
    for fn in ("mtlattn_varlen_fwd_workspace_size", "mtlattn_varlen_bwd_workspace_size"):
        getattr(L, fn).restype = ctypes.c_size_t
        getattr(L, fn).argtypes = [ctypes.POINTER(Problem)]
    L.mtlattn_attn_splitkv_workspace_size.restype = ctypes.c_size_t
    L.mtlattn_attn_splitkv_workspace_size.argtypes = [ctypes.POINTER(Problem), ctypes.c_int32]
    L.mtlattn_decode_num_splits.restype = ctypes.c_int32
    L.mtlattn_decode_num_splits.argtypes = [ctypes.POINTER(Problem)]
    i64, vp = ctypes.c_int64, ctypes.c_void_p
    L.mtlattn_paged_decode_workspace_size.restype = ctypes.c_size_t
    L.mtlattn_paged_decode_workspace_size.argtypes = [ctypes.POINTER(Problem), i64]
    L.mtlattn_paged_decode.argtypes = [ctypes.POINTER(Problem), vp, i64, vp, i64, vp, i64, ctypes.c_int32, i64, vp,
                                       i64, i64, vp, vp, vp, ctypes.c_size_t, vp]
    return L


FAKE = ctypes.c_void_p(0x1000)   # never dereferenced: every call below stops in validation


def problem(**kw):
    p = Problem(dtype=BF16, num_seqs=2, total_q=64, total_kv=64, num_heads_q=8, num_heads_kv=2,
                head_dim=128, max_seqlen_q=32, scale=0.088, causal=1, window=0,
                cu_seqlens_q=FAKE, cu_seqlens_kv=FAKE, bias=None, bias_q_stride=0, bias_h_stride=0,
                bias_kv_cols=0)
    for k, v in kw.items():
        setattr(p, k, v)
    return p


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(mtlattn_\w+)\s*\(", text)))


def test_exports_every_declared_function(lib):
    names = declared_functions()
    assert len(names) >= 12
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/mtlattn_capi.h but not exported"


def test_abi_version(lib):
    m = re.search(r"#define MTLATTN_ABI_VERSION (\d+)", open(HEADER).read())
    assert lib.mtlattn_abi_version() == int(m.group(1))


def _fwd(lib, p):
    return lib.mtlattn_varlen_fwd(ctypes.byref(p), FAKE, ctypes.c_int64(3072), FAKE, ctypes.c_int64(768), FAKE,
                                  ctypes.c_int64(768), FAKE, None, None, ctypes.c_size_t(0), None)


@pytest.mark.parametrize("kw,msg", [
    (dict(num_heads_q=6, num_heads_kv=4), "multiple of kv heads"),
    (dict(head_dim=300), "head_dim 300 unsupported"),
    (dict(dtype=7), "unsupported dtype"),
    (dict(num_seqs=0), "[B+1]"),
    (dict(cu_seqlens_q=None), "cu_seqlens"),
    (dict(total_q=-1), "negative token count"),
    (dict(bias=FAKE, bias_q_stride=-5), "strides must be non-negative"),
])
def test_forward_validation(lib, kw, msg):
    rc = _fwd(lib, problem(**kw))
    assert rc == ERR_INVALID
    assert msg in lib.mtlattn_last_error().decode()


def test_null_problem(lib):
    assert lib.mtlattn_varlen_fwd(None, FAKE, 0, FAKE, 0, FAKE, 0, FAKE, None, None, 0, None) == ERR_INVALID
    assert b"null problem" in lib.mtlattn_last_error()


def test_empty_query_is_a_no_op(lib):
    assert _fwd(lib, problem(total_q=0)) == OK
    assert lib.mtlattn_last_error() == b""


def test_null_tensor_pointer(lib):
    p = problem()
    rc = lib.mtlattn_varlen_fwd(ctypes.byref(p), None, 0, FAKE, 0, FAKE, 0, FAKE, None, None, 0, None)
    assert rc == ERR_INVALID and b"null" in lib.mtlattn_last_error()


def _splitkv_bytes(rows, d):
    o = rows * d * 4
    return ((o + 255) // 256) * 256 + rows * 4


def test_workspace_sizes(lib):
    p = problem(total_q=1000, num_heads_q=32, num_heads_kv=8)
    assert lib.mtlattn_varlen_bwd_workspace_size(ctypes.byref(p)) == 1000 * 32 * 4
    # explicit splits: 16 partial rows per (kv head, head group, sequence, split);
    # max_seqlen_q = 32 leaves one head per 16-row group, so g = 4 groups
    n = lib.mtlattn_attn_splitkv_workspace_size(ctypes.byref(p), 4)
    assert n == _splitkv_bytes(8 * 4 * (2 * 4) * 16, 128)
    assert lib.mtlattn_attn_splitkv_workspace_size(ctypes.byref(p), 0) == 0


def test_fp32_split_workspace_sizes(lib):
    """fp32 problems on the fp32 matrix-core kernels whose grids (one
    workgroup per 128 rows and head) would leave CUs idle ask for split
    partials (256 CUs assumed without a GPU, as on MI355X): the forward for
    normalised O and LSE per split, the backward after delta (256-byte
    aligned) for the larger of dQ's and dK/dV's partials. Large grids, 16-bit
    inputs and head dims the fp32 matrix-core kernels do not take ask for
    none; the forward's split count is capped so its partials fit the 64 MiB
    no-allocation scratch."""
    # C1: 460 rows, 4 + 4 heads, D = 64, 4 sequences: 16 workgroups -> 8 splits
    p = problem(dtype=F32, num_seqs=4, total_q=460, total_kv=460, num_heads_q=4, num_heads_kv=4, head_dim=64,
                max_seqlen_q=250)
    assert lib.mtlattn_varlen_fwd_workspace_size(ctypes.byref(p)) == 8 * 460 * 4 * (64 + 1) * 4
    delta = 460 * 4 * 4
    dq_part = 8 * 460 * 4 * 64 * 4
    dkv_part = 8 * 2 * 460 * 4 * 64 * 4
    assert lib.mtlattn_varlen_bwd_workspace_size(ctypes.byref(p)) == (delta + 255) // 256 * 256 + max(dq_part, dkv_part)
    # a grid that fills the GPU: no splits
    p = problem(dtype=F32, num_seqs=8, total_q=8 * 4096, total_kv=8 * 4096, num_heads_q=32, num_heads_kv=8,
                head_dim=128, max_seqlen_q=4096)
    assert lib.mtlattn_varlen_fwd_workspace_size(ctypes.byref(p)) == 0
    assert lib.mtlattn_varlen_bwd_workspace_size(ctypes.byref(p)) == 8 * 4096 * 32 * 4
    # the same small shape in bf16, or at an fp32 head dim of the portable kernels: none
    for kw in ({"dtype": BF16, "head_dim": 64}, {"dtype": F32, "head_dim": 160}, {"dtype": F32, "head_dim": 66}):
        p = problem(num_seqs=4, total_q=460, total_kv=460, num_heads_q=4, num_heads_kv=4, max_seqlen_q=250, **kw)
        assert lib.mtlattn_varlen_fwd_workspace_size(ctypes.byref(p)) == 0, kw
        assert lib.mtlattn_varlen_bwd_workspace_size(ctypes.byref(p)) == 460 * 4 * 4, kw
    # 511 workgroups would split 2 ways, but 2 x 33.75 MB of forward partials
    # exceed the 64 MiB scratch: the forward stays unsplit
    p = problem(dtype=F32, num_seqs=1, total_q=73 * 128, total_kv=73 * 128, num_heads_q=7, num_heads_kv=7,
                head_dim=128, max_seqlen_q=73 * 128)
    assert 2 * 73 * 128 * 7 * 129 * 4 > 64 << 20
    assert lib.mtlattn_varlen_fwd_workspace_size(ctypes.byref(p)) == 0


def test_backward_workspace_checked(lib):
    p = problem()
    rc = lib.mtlattn_varlen_bwd(ctypes.byref(p), FAKE, 0, FAKE, 0, FAKE, 0, FAKE, 0, FAKE, 0, FAKE, FAKE, FAKE, FAKE,
                                None, ctypes.c_size_t(16), None)
    assert rc == ERR_WORKSPACE and b"workspace too small" in lib.mtlattn_last_error()


def _c5_like(**kw):
    base = dict(dtype=BF16, num_seqs=64, total_q=64, total_kv=64 * 36864, num_heads_q=64, num_heads_kv=8,
                head_dim=128, max_seqlen_q=1, causal=1)
    base.update(kw)
    return problem(**base)


def test_decode_routing(lib, monkeypatch):
    """Reference gate (src/ext.mm:372-376): few queries, long KV, fp16/bf16,
    D in {64,128}; unlike the reference, a bias or a window (whose band is
    long enough) is routed too."""
    monkeypatch.delenv("MTLATTN_NO_SPLITKV", raising=False)
    monkeypatch.delenv("MTLATTN_NO_MPP", raising=False)
    monkeypatch.delenv("MTLATTN_NO_MFMA", raising=False)
    slots = lib.mtlattn_decode_num_splits(ctypes.byref(_c5_like()))
    # fixed KV chunks: slots = total_kv / chunk + num_seqs + 1 with a chunk of
    # >= 256 keys sized for ~18 work items per CU (256 CUs without a device),
    # rounded to the nearest multiple of 256
    total_kv = 64 * 36864
    chunk = -(-(total_kv * 8) // (256 * 18))
    chunk = (chunk + 128) // 256 * 256
    assert slots == total_kv // chunk + 64 + 1
    # 8 kv heads x 1 head group (8 heads x q_len 1 fill a 16-row group)
    assert lib.mtlattn_varlen_fwd_workspace_size(ctypes.byref(_c5_like())) == _splitkv_bytes(8 * slots * 16, 128)
    for kw in (dict(dtype=F32), dict(head_dim=96), dict(window=128), dict(max_seqlen_q=17),
               dict(total_kv=64 * 2000)):
        assert lib.mtlattn_decode_num_splits(ctypes.byref(_c5_like(**kw))) == 0, kw
    # a bias changes nothing in the split plan
    assert lib.mtlattn_decode_num_splits(ctypes.byref(_c5_like(bias=FAKE, bias_kv_cols=10))) == slots
    # a window: equal splits of the band (W + q_len - 1 keys, plus up to 31
    # below it for the tile-aligned start) per sequence, the split length
    # sized like the chunk for the band's work (64 sequences x 4096 keys)
    c = -(-(64 * 4096 * 8) // (256 * 18))
    c = (c + 128) // 256 * 256
    ns = -(-(4096 + 31) // c)
    assert lib.mtlattn_decode_num_splits(ctypes.byref(_c5_like(window=4096))) == 64 * ns
    assert lib.mtlattn_varlen_fwd_workspace_size(ctypes.byref(_c5_like(window=4096))) == \
        _splitkv_bytes(8 * 64 * ns * 16, 128)
    monkeypatch.setenv("MTLATTN_NO_SPLITKV", "1")
    assert lib.mtlattn_decode_num_splits(ctypes.byref(_c5_like())) == 0


def test_splitkv_entry_validation(lib):
    p = problem(dtype=F32, max_seqlen_q=1)
    rc = lib.mtlattn_attn_splitkv(ctypes.byref(p), FAKE, 0, FAKE, 0, FAKE, 0, FAKE, None, 2, None, 0, None)
    assert rc == ERR_UNSUPPORTED and b"half/bf16" in lib.mtlattn_last_error()
    p = problem(max_seqlen_q=17)
    rc = lib.mtlattn_attn_splitkv(ctypes.byref(p), FAKE, 0, FAKE, 0, FAKE, 0, FAKE, None, 2, None, 0, None)
    assert rc == ERR_UNSUPPORTED
    # a window passes validation (the split path honours it): the empty
    # workspace is what fails
    p = problem(max_seqlen_q=1, window=4)
    rc = lib.mtlattn_attn_splitkv(ctypes.byref(p), FAKE, 0, FAKE, 0, FAKE, 0, FAKE, None, 2, None, 0, None)
    assert rc == ERR_WORKSPACE
    p = problem(max_seqlen_q=1)
    rc = lib.mtlattn_attn_splitkv(ctypes.byref(p), FAKE, 0, FAKE, 0, FAKE, 0, FAKE, None, 0, None, 0, None)
    assert rc == ERR_INVALID


def test_paged_decode_validation(lib):
    """Paged decode (no reference counterpart): argument checks before any
    launch, and the workspace is the equal-split plan's size."""
    args = lambda p, ps=16, pages=8, bt=FAKE, bts=4: (ctypes.byref(p), FAKE, 0, FAKE, 0, FAKE, 0, ps, pages, bt, bts,
                                                      4096, FAKE, None, None, 0, None)   # noqa: E731
    p = problem(max_seqlen_q=1)
    assert lib.mtlattn_paged_decode(*args(p, ps=24)) == ERR_INVALID
    assert b"multiple of 16" in lib.mtlattn_last_error()
    assert lib.mtlattn_paged_decode(*args(p, ps=0)) == ERR_INVALID
    assert lib.mtlattn_paged_decode(*args(p, pages=0)) == ERR_INVALID
    assert lib.mtlattn_paged_decode(*args(p, bts=0)) == ERR_INVALID
    assert lib.mtlattn_paged_decode(*args(p, bt=None)) == ERR_INVALID
    assert lib.mtlattn_paged_decode(*args(problem(max_seqlen_q=17))) == ERR_UNSUPPORTED
    assert lib.mtlattn_paged_decode(*args(problem(max_seqlen_q=1, head_dim=96))) == ERR_UNSUPPORTED
    assert lib.mtlattn_paged_decode(*args(problem(max_seqlen_q=1, dtype=F32))) == ERR_UNSUPPORTED
    # valid arguments: the empty workspace is what fails
    assert lib.mtlattn_paged_decode(*args(p)) == ERR_WORKSPACE
    # fixed chunks for p.total_kv = 64 keys (bound on the logical total): a
    # 256-key chunk, slots 64 // 256 + 2 + 1 per (kv head x 1 head group)
    assert lib.mtlattn_paged_decode_workspace_size(ctypes.byref(p), 4096) == _splitkv_bytes(2 * 3 * 16, 128)
    # with a window: equal splits of the band (W + q_len - 1 + 31 keys)
    pw = problem(max_seqlen_q=1, window=1000)
    c = -(-(2 * 1031 * 2) // (256 * 18))
    c = max(256, (c + 128) // 256 * 256)
    ns = -(-1031 // c)
    assert lib.mtlattn_paged_decode_workspace_size(ctypes.byref(pw), 4096) == _splitkv_bytes(2 * 2 * ns * 16, 128)


def test_dq_dtype_checked(lib):
    p = problem()
    rc = lib.mtlattn_bwd_dq(ctypes.byref(p), FAKE, 0, FAKE, 0, FAKE, 0, FAKE, 0, FAKE, FAKE, FAKE, F16, None)
    assert rc == ERR_INVALID and b"dq dtype" in lib.mtlattn_last_error()


def test_ctypes_binding_covers_header():
    """mtlattn_amd/capi.py declares every function of the header, with the
    header's parameter count."""
    from mtlattn_amd import capi
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decl = dict(re.findall(r"\b(mtlattn_\w+)\s*\(([^)]*)\)\s*;", text))
    assert set(decl) == set(capi.SIGNATURES)
    for name, params in decl.items():
        n = 0 if params.strip() in ("", "void") else params.count(",") + 1
        assert len(capi.SIGNATURES[name][1]) == n, name
    assert capi.lib().mtlattn_abi_version() == capi.ABI_VERSION
