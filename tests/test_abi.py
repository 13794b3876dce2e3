"""The C ABI of libsiq_kernels.so, exercised on the CPU: every symbol the
header declares is exported, and host-side validation rejects bad arguments
with the documented status before anything reaches the GPU."""

import re
from pathlib import Path

import pytest

from siq_vl_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "siq_kernels.h"
FAKE = 0x10000  # 16-byte aligned, never dereferenced: validation fails first


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return sorted(set(re.findall(r"\b(siq_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_bound_symbols():
    assert declared_symbols() == sorted(_lib.EXPORTED)


def test_library_exports_every_declared_symbol(lib):
    for name in declared_symbols():
        assert hasattr(lib, name), name


def test_abi_version(lib):
    m = re.search(r"#define\s+SIQ_ABI_VERSION\s+(\d+)", HEADER.read_text())
    assert m and lib.siq_abi_version() == int(m.group(1))


def test_status_codes_match_header():
    text = HEADER.read_text()
    for name in ("SIQ_OK", "SIQ_ERR_INVALID_ARGUMENT", "SIQ_ERR_UNSUPPORTED", "SIQ_ERR_WORKSPACE",
                 "SIQ_ERR_ALIGNMENT", "SIQ_ERR_LAUNCH"):
        m = re.search(name + r"\s*=\s*(-?\d+)", text)
        assert m, name
        assert int(m.group(1)) == getattr(_lib, name)


def test_workspace_sizes(lib):
    f = lib.siq_attn_fwd_workspace_bytes
    b = lib.siq_attn_bwd_workspace_bytes
    assert f(-1, 10, 10, 2, 1, 64) == 0 and b(2, 10, 10, 0, 1, 64, 1) == 0
    small, big = f(4, 1000, 1000, 12, 2, 128), f(64, 100000, 100000, 12, 2, 128)
    assert 0 < small < big
    assert b(4, 1000, 1000, 12, 2, 128, 1) > f(4, 1000, 1000, 12, 2, 128)  # bwd adds Delta
    # the atomic backward adds its fp32 dQ sums, [total_q, hq, d]
    assert b(4, 1000, 1000, 12, 2, 128, 0) - b(4, 1000, 1000, 12, 2, 128, 1) >= 1000 * 12 * 128 * 4
    assert f(4, 1000, 1000, 12, 2, 128) % 16 == 0
    w = lib.siq_flce_workspace_bytes
    assert w(-1, 64, 64, 8, 1) == 0
    a, c = w(16384, 1536, 151936, 8192, 1), w(16384, 1536, 151936, 2048, 1)
    assert a > c > 0  # chunk bounds the logits-sized scratch
    # never a full [n, V] fp32 logits buffer
    assert a < 16384 * 151936 * 4


def test_flce_default_workspace_bound_at_config4(lib):
    """Config 4 at the default chunk: the softmax-numerator buffer stays within
    its 2 GiB budget, below the bf16 logits of the batch (4.98 GB), and the
    whole workspace (numerators, tile max / sum, split-K dH partials, the fp32
    dW accumulator, compacted rows) within 4 GiB."""
    from siq_vl_amd import cross_entropy as C

    n, hdim, vocab = 16384, 1536, 151936
    chunk = C.default_chunk_tokens(vocab)
    assert chunk % 256 == 0 and 2 * chunk * vocab <= C.DEFAULT_E_BUDGET_BYTES
    assert chunk == 6912
    total = lib.siq_flce_workspace_bytes(n, hdim, vocab, chunk, 1)
    one_chunk = lib.siq_flce_workspace_bytes(n, hdim, vocab, n, 1)
    assert total <= 4 << 30, total
    assert total < 2 * n * vocab  # the bf16 logits alone
    assert one_chunk - total > (2 * (n - chunk) * vocab) // 2  # the bound is what shrank it
    assert C.flce_workspace_bytes(n, hdim, vocab, None, True) == total
    # loss only: no numerators at all
    assert lib.siq_flce_loss_workspace_bytes(n, hdim, vocab) < 128 << 20


def test_flce_fp32_dw_sum_only_beyond_two_chunks(lib):
    """Over at most two chunks dW is summed in dW itself (bf16), so the
    workspace holds the fp32 [vocab, hdim] sum only when the rows may span a
    third chunk: one row more than two chunks adds exactly that buffer (plus
    the per-row pieces of one more row)."""
    hdim, vocab, chunk = 256, 4096, 512
    w = lib.siq_flce_workspace_bytes
    two, three = w(2 * chunk, hdim, vocab, chunk, 1), w(2 * chunk + 1, hdim, vocab, chunk, 1)
    fp32_sum = vocab * hdim * 4
    assert fp32_sum <= three - two < fp32_sum + 4096 + 256 * (hdim * 2 + 16)
    # without dweight there is no sum either way
    assert w(2 * chunk + 1, hdim, vocab, chunk, 0) - w(2 * chunk, hdim, vocab, chunk, 0) < fp32_sum
    # one chunk or two: no fp32 sum
    assert w(2 * chunk, hdim, vocab, chunk, 1) - w(2 * chunk, hdim, vocab, chunk, 0) < fp32_sum


def test_plan_sizes(lib):
    assert lib.siq_attn_plan_bytes(-1, 10, 10) == 0
    a, b = lib.siq_attn_plan_bytes(32, 16384, 16384), lib.siq_attn_plan_bytes(200, 32768, 32768)
    assert 0 < a < b and a % 256 == 0
    # the backward call's workspace is a plan plus the backward's own scratch
    for det in (1, 0):
        full = lib.siq_attn_bwd_workspace_bytes(32, 16384, 16384, 12, 2, 128, det)
        own = lib.siq_attn_bwd_plan_workspace_bytes(32, 16384, 16384, 12, 2, 128, det)
        assert full == a + own


def _strides(n=16):
    return _lib.int64_array([128] * n)


def _attn_fwd(lib, **kw):
    args = dict(q=FAKE, k=FAKE, v=FAKE, o=FAKE, lse=FAKE, cu_q=FAKE, cu_k=FAKE, batch=2, max_q=8, max_k=8,
                total_q=16, total_k=16, hq=4, hkv=2, d=128, strides=_strides(8), scale=0.1, causal=1, ws=None,
                ws_bytes=0, stream=None)
    args.update(kw)
    return lib.siq_attn_varlen_fwd(*args.values())


@pytest.mark.parametrize("kw,code", [
    (dict(d=96), _lib.SIQ_ERR_UNSUPPORTED),
    (dict(hq=3), _lib.SIQ_ERR_INVALID_ARGUMENT),
    (dict(hkv=0), _lib.SIQ_ERR_INVALID_ARGUMENT),
    (dict(batch=-1), _lib.SIQ_ERR_INVALID_ARGUMENT),
    (dict(total_q=1 << 31), _lib.SIQ_ERR_INVALID_ARGUMENT),
    (dict(scale=float("nan")), _lib.SIQ_ERR_INVALID_ARGUMENT),
    (dict(cu_q=None), _lib.SIQ_ERR_INVALID_ARGUMENT),
    (dict(strides=None), _lib.SIQ_ERR_INVALID_ARGUMENT),
    (dict(q=FAKE + 8), _lib.SIQ_ERR_ALIGNMENT),
    (dict(v=None), _lib.SIQ_ERR_INVALID_ARGUMENT),
    (dict(lse=FAKE + 2), _lib.SIQ_ERR_ALIGNMENT),
    (dict(ws=None), _lib.SIQ_ERR_WORKSPACE),
    (dict(ws=FAKE, ws_bytes=16), _lib.SIQ_ERR_WORKSPACE),
])
def test_attention_fwd_validation(lib, kw, code):
    assert _attn_fwd(lib, **kw) == code
    assert lib.siq_last_error().decode()


def test_attention_fwd_odd_strides_rejected(lib):
    st = _lib.int64_array([128, 128, 130, 128, 128, 128, 128, 128])
    assert _attn_fwd(lib, strides=st) == _lib.SIQ_ERR_ALIGNMENT


def test_attention_empty_batch_is_a_no_op(lib):
    # nothing to compute: returns before touching the device
    assert _attn_fwd(lib, batch=0, total_q=0, total_k=0, q=None, k=None, v=None, o=None, lse=None) == _lib.SIQ_OK


def test_attention_bwd_validation(lib):
    for det in (1, 0):
        rc = lib.siq_attn_varlen_bwd(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 2, 8, 8, 16,
                                     16, 4, 2, 64, _strides(16), 0.1, 1, det, FAKE, 8, None)
        assert rc == _lib.SIQ_ERR_WORKSPACE
        rc = lib.siq_attn_varlen_bwd(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None, FAKE, FAKE, FAKE, FAKE, 2, 8, 8, 16,
                                     16, 4, 2, 64, _strides(16), 0.1, 1, det, None, 0, None)
        assert rc == _lib.SIQ_ERR_INVALID_ARGUMENT and b"dq" in lib.siq_last_error()
    # the atomic backward's workspace is checked against its own (larger) size
    need_det = lib.siq_attn_bwd_workspace_bytes(2, 16, 16, 4, 2, 64, 1)
    rc = lib.siq_attn_varlen_bwd(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 2, 8, 8, 16, 16,
                                 4, 2, 64, _strides(16), 0.1, 1, 0, FAKE, need_det, None)
    assert rc == _lib.SIQ_ERR_WORKSPACE


def test_plan_entry_validation(lib):
    bp = lib.siq_attn_build_plan
    assert bp(FAKE, FAKE, 2, 16, 16, 4, 2, 1, None, 0, None) == _lib.SIQ_ERR_WORKSPACE
    assert bp(None, FAKE, 2, 16, 16, 4, 2, 1, FAKE, 1 << 20, None) == _lib.SIQ_ERR_INVALID_ARGUMENT
    assert bp(FAKE, FAKE, 2, 16, 16, 3, 2, 1, FAKE, 1 << 20, None) == _lib.SIQ_ERR_INVALID_ARGUMENT
    need = lib.siq_attn_plan_bytes(2, 16, 16)
    fwd = lib.siq_attn_varlen_fwd_plan
    assert fwd(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 16, 16, 4, 2, 128, _strides(8), 0.1, 1, FAKE, need - 16,
               None) == _lib.SIQ_ERR_WORKSPACE
    assert fwd(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 16, 16, 4, 2, 96, _strides(8), 0.1, 1, FAKE, need,
               None) == _lib.SIQ_ERR_UNSUPPORTED
    assert fwd(None, None, None, None, None, 0, 0, 0, 4, 2, 128, _strides(8), 0.1, 1, None, 0, None) == _lib.SIQ_OK
    bwd = lib.siq_attn_varlen_bwd_plan
    for det in (1, 0):
        own = lib.siq_attn_bwd_plan_workspace_bytes(2, 16, 16, 4, 2, 128, det)
        assert bwd(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 2, 16, 16, 4, 2, 128, _strides(16), 0.1, 1,
                   det, FAKE, need, FAKE, own - 16, None) == _lib.SIQ_ERR_WORKSPACE
        assert bwd(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 2, 16, 16, 4, 2, 128, _strides(16), 0.1, 1,
                   det, None, need, FAKE, own, None) == _lib.SIQ_ERR_WORKSPACE


def test_flce_loss_validation(lib):
    f = lib.siq_flce_loss
    need = lib.siq_flce_loss_workspace_bytes(16, 128, 1024)
    assert f(FAKE, FAKE, FAKE, 16, 128, 1024, -100, 0, None, FAKE, FAKE, FAKE, FAKE, need - 256,
             None) == _lib.SIQ_ERR_WORKSPACE
    assert f(None, FAKE, FAKE, 16, 128, 1024, -100, 0, None, FAKE, FAKE, FAKE, FAKE, need,
             None) == _lib.SIQ_ERR_INVALID_ARGUMENT
    assert f(FAKE, FAKE, FAKE, 16, 100, 1024, -100, 0, None, FAKE, FAKE, FAKE, FAKE, need,
             None) == _lib.SIQ_ERR_UNSUPPORTED
    assert f(FAKE, FAKE, FAKE, 16, 128, 1024, -100, 1, None, FAKE, FAKE, FAKE, FAKE, need,
             None) == _lib.SIQ_ERR_INVALID_ARGUMENT


def _flce(lib, **kw):
    args = dict(hidden=FAKE, weight=FAKE, labels=FAKE, n=16, hdim=128, vocab=1024, ignore_index=-100, reduction=0,
                divisor=None, loss=FAKE, count=FAKE, bad=FAKE, dh=FAKE, dw=FAKE, chunk=8, ws=None, ws_bytes=0,
                stream=None)
    args.update(kw)
    return lib.siq_flce_fwd_bwd(*args.values())


@pytest.mark.parametrize("kw,code", [
    (dict(hdim=100), _lib.SIQ_ERR_UNSUPPORTED),
    (dict(vocab=1001), _lib.SIQ_ERR_UNSUPPORTED),
    (dict(n=-1), _lib.SIQ_ERR_INVALID_ARGUMENT),
    (dict(reduction=2), _lib.SIQ_ERR_INVALID_ARGUMENT),
    (dict(reduction=1), _lib.SIQ_ERR_INVALID_ARGUMENT),
    (dict(loss=None), _lib.SIQ_ERR_INVALID_ARGUMENT),
    (dict(labels=None), _lib.SIQ_ERR_INVALID_ARGUMENT),
    (dict(hidden=FAKE + 4), _lib.SIQ_ERR_ALIGNMENT),
    (dict(weight=None), _lib.SIQ_ERR_ALIGNMENT),
    (dict(chunk=0), _lib.SIQ_ERR_INVALID_ARGUMENT),
    (dict(ws=FAKE, ws_bytes=64), _lib.SIQ_ERR_WORKSPACE),
])
def test_flce_validation(lib, kw, code):
    assert _flce(lib, **kw) == code
    assert lib.siq_last_error().decode()


def test_scale_validation(lib):
    assert lib.siq_scale_bf16_inplace(None, 0, None, None) == _lib.SIQ_OK
    assert lib.siq_scale_bf16_inplace(None, -1, None, None) == _lib.SIQ_ERR_INVALID_ARGUMENT
    assert lib.siq_scale_bf16_inplace(FAKE + 2, 8, FAKE, None) == _lib.SIQ_ERR_ALIGNMENT
    assert lib.siq_scale_bf16(FAKE, None, 8, FAKE, None) == _lib.SIQ_ERR_INVALID_ARGUMENT
    assert lib.siq_scale_bf16(FAKE, FAKE + 8, 8, FAKE, None) == _lib.SIQ_ERR_ALIGNMENT
    assert lib.siq_scale_bf16(None, None, 0, None, None) == _lib.SIQ_OK


def test_check_maps_status_to_exceptions():
    with pytest.raises(ValueError):
        _lib.check(_lib.SIQ_ERR_INVALID_ARGUMENT, "x")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.SIQ_ERR_LAUNCH, "x")
    _lib.check(_lib.SIQ_OK, "x")


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_LIB", None)
    monkeypatch.setenv("SIQ_KERNELS_LIB", str(tmp_path / "absent.so"))
    with pytest.raises(RuntimeError, match="build"):
        _lib.lib()


def test_ctypes_prototypes_cover_header_arity():
    """Each bound prototype has the parameter count of its header declaration."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    for name, (_, args) in _lib._PROTOS.items():
        m = re.search(r"\b" + name + r"\s*\(([^)]*)\)", text)
        assert m, name
        params = [p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"]
        assert len(params) == len(args), (name, len(params), len(args))


def _rope(lib, fwd=True, **kw):
    args = dict(x0=FAKE, x1=FAKE, cos=FAKE, sin=FAKE, y0=FAKE, y1=FAKE, batch=1, seqlen=8, hq=4, hkv=2, d=128,
                strides=_strides(16), stream=None)
    args.update(kw)
    fn = lib.siq_rope_fwd if fwd else lib.siq_rope_bwd
    return fn(*args.values())


@pytest.mark.parametrize("fwd", [True, False])
@pytest.mark.parametrize("kw,code", [
    (dict(d=72), _lib.SIQ_ERR_UNSUPPORTED),
    (dict(d=0), _lib.SIQ_ERR_UNSUPPORTED),
    (dict(d=1024), _lib.SIQ_ERR_UNSUPPORTED),
    (dict(hq=-1), _lib.SIQ_ERR_INVALID_ARGUMENT),
    (dict(hkv=-1), _lib.SIQ_ERR_INVALID_ARGUMENT),
    (dict(hkv=0), _lib.SIQ_ERR_INVALID_ARGUMENT),
    (dict(hq=5000), _lib.SIQ_ERR_INVALID_ARGUMENT),
    (dict(batch=1 << 20, seqlen=1 << 12), _lib.SIQ_ERR_INVALID_ARGUMENT),
    (dict(batch=-1), _lib.SIQ_ERR_INVALID_ARGUMENT),
    (dict(seqlen=-3), _lib.SIQ_ERR_INVALID_ARGUMENT),
    (dict(strides=None), _lib.SIQ_ERR_INVALID_ARGUMENT),
    (dict(cos=None), _lib.SIQ_ERR_INVALID_ARGUMENT),
    (dict(y1=None), _lib.SIQ_ERR_INVALID_ARGUMENT),
    (dict(x0=FAKE + 8), _lib.SIQ_ERR_ALIGNMENT),
    (dict(sin=FAKE + 4), _lib.SIQ_ERR_ALIGNMENT),
])
def test_rope_validation(lib, fwd, kw, code):
    assert _rope(lib, fwd, **kw) == code
    assert lib.siq_last_error().decode()


@pytest.mark.parametrize("pos", [0, 5, 7, 15])
def test_rope_odd_strides_rejected(lib, pos):
    st = [128] * 16
    st[pos] = 132
    assert _rope(lib, strides=_lib.int64_array(st)) == _lib.SIQ_ERR_ALIGNMENT
    st[pos] = -128
    assert _rope(lib, strides=_lib.int64_array(st)) == _lib.SIQ_ERR_ALIGNMENT


def test_rope_k_only_pass_validation(lib):
    # hq = 0: q and its output are not read (may be NULL); k, cos, sin and k's output still are
    assert _rope(lib, hq=0, x0=None, y0=None, seqlen=0) == _lib.SIQ_OK
    assert _rope(lib, hq=0, x0=None, y0=None, x1=None) == _lib.SIQ_ERR_INVALID_ARGUMENT
    assert _rope(lib, False, hq=0, x0=None, y0=None, y1=FAKE + 8) == _lib.SIQ_ERR_ALIGNMENT


def test_rope_attention_entry_validation(lib):
    need = lib.siq_attn_plan_bytes(2, 16, 16)
    f = lib.siq_attn_rope_fwd_plan
    st = _strides(12)
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None, FAKE, 2, 16, 16, 4, 2, 128, st, 0.1, 1, FAKE, need,
             None) == _lib.SIQ_ERR_INVALID_ARGUMENT
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE + 8, FAKE, 2, 16, 16, 4, 2, 128, st, 0.1, 1, FAKE, need,
             None) == _lib.SIQ_ERR_ALIGNMENT
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, None, FAKE, FAKE, 2, 16, 16, 4, 2, 128, st, 0.1, 1, FAKE, need,
             None) == _lib.SIQ_ERR_INVALID_ARGUMENT
    bad = [128] * 12
    bad[10] = 132
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 2, 16, 16, 4, 2, 128, _lib.int64_array(bad), 0.1, 1, FAKE,
             need, None) == _lib.SIQ_ERR_ALIGNMENT
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 2, 16, 16, 4, 2, 128, st, 0.1, 1, FAKE, need - 16,
             None) == _lib.SIQ_ERR_WORKSPACE
    b = lib.siq_attn_rope_bwd_plan
    own = lib.siq_attn_bwd_plan_workspace_bytes(2, 16, 16, 4, 2, 128, 1)
    assert b(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None, 2, 16, 16, 4, 2, 128, _strides(18),
             0.1, 1, FAKE, need, FAKE, own, None) == _lib.SIQ_ERR_INVALID_ARGUMENT
    assert b(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 2, 16, 16, 4, 2, 128, _strides(18),
             0.1, 1, FAKE, need, FAKE, own - 16, None) == _lib.SIQ_ERR_WORKSPACE


def test_rope_empty_is_a_no_op(lib):
    # nothing to rotate: returns before touching the device (pointers are never read)
    assert _rope(lib, seqlen=0) == _lib.SIQ_OK
    assert _rope(lib, False, batch=0) == _lib.SIQ_OK


def test_embedding_bwd_validation(lib):
    """siq_embedding_bwd rejects bad arguments before any launch (CPU: no
    device pointer is ever dereferenced)."""
    ws_need = lib.siq_embedding_bwd_workspace_bytes(100, 1000)
    assert ws_need > 100 * 8 and lib.siq_embedding_bwd_workspace_bytes(-1, 1000) == 0
    assert lib.siq_embedding_bwd_workspace_bytes(0, 1000) > 0
    base = dict(grad=FAKE, ids=FAKE, n=100, vocab=1000, hidden=64, dtype=0, s0=5, s1=-1, dw=FAKE, ws=FAKE,
                ws_bytes=ws_need)

    def call(**kw):
        a = dict(base, **kw)
        return lib.siq_embedding_bwd(a["grad"], a["ids"], a["n"], a["vocab"], a["hidden"], a["dtype"], a["s0"],
                                     a["s1"], a["dw"], a["ws"], a["ws_bytes"], None)

    assert call(n=-1) == _lib.SIQ_ERR_INVALID_ARGUMENT
    assert call(vocab=0) == _lib.SIQ_ERR_INVALID_ARGUMENT
    assert call(hidden=60) == _lib.SIQ_ERR_UNSUPPORTED
    assert call(dtype=2) == _lib.SIQ_ERR_INVALID_ARGUMENT
    assert call(dw=None) == _lib.SIQ_ERR_ALIGNMENT
    assert call(dw=FAKE + 8) == _lib.SIQ_ERR_ALIGNMENT
    assert call(grad=None) == _lib.SIQ_ERR_INVALID_ARGUMENT
    assert call(ws_bytes=ws_need - 1) == _lib.SIQ_ERR_WORKSPACE
    assert call(ws=None) == _lib.SIQ_ERR_WORKSPACE
    assert "workspace" in lib.siq_last_error().decode()
