"""CPU: the C ABI library loads, exports everything ``include/asrattn.h``
declares, and the ctypes mirrors of its structs match the C layout.

No kernel is launched here; argument checks that fail before any device work
are exercised through the real library.
"""

from __future__ import annotations

import ctypes
import re
import subprocess

import pytest

from conftest import ROOT

HEADER = ROOT / "include" / "asrattn.h"


def declared_functions() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"^\w[\w\s\*]*?\b(asrattn_\w+)\s*\(", text, flags=re.M))


@pytest.fixture(scope="module")
def lib():
    import torch  # noqa: F401  (the library binds to torch's HIP runtime)
    from asrback_amd import _lib

    if not _lib.LIBRARY.is_file():
        from asrback_amd import build

        build.build()
    return _lib.load()


def test_header_declares_expected_entry_points():
    assert declared_functions() == {
        "asrattn_fwd",
        "asrattn_fwd_fsmn",
        "asrattn_decode",
        "asrattn_decode_noalloc",
        "asrattn_decode_append",
        "asrattn_decode_paged",
        "asrattn_local",
        "asrattn_choose",
        "asrattn_choose_workspace_size",
        "asrattn_decode_workspace_size",
        "asrattn_decode_num_splits",
        "asrattn_last_error",
        "asrattn_abi_version",
    }


def test_library_exports_every_declared_symbol(lib):
    from asrback_amd import _lib

    for name in declared_functions():
        assert hasattr(lib, name), name
    assert set(_lib.SIGNATURES) == declared_functions()


def test_library_is_gfx950_and_binds_torch_runtime(lib):
    from asrback_amd import _lib

    maps = open("/proc/self/maps").read()
    runtimes = {line.split()[-1] for line in maps.splitlines() if "libamdhip64" in line}
    assert len(runtimes) == 1, runtimes  # one HIP runtime in the process: torch's
    assert lib.asrattn_abi_version() == _lib.ABI_VERSION


def _c_layout(struct: str, fields: list[str]) -> dict[str, int]:
    """sizeof and offsetof as the C compiler lays the header's struct out."""
    lines = [f'printf("sizeof %zu\\n", sizeof({struct}));']
    lines += [f'printf("{f} %zu\\n", offsetof({struct}, {f}));' for f in fields]
    source = (
        "#include <stddef.h>\n#include <stdio.h>\n#include \"asrattn.h\"\n"
        "int main(void) {\n" + "\n".join(lines) + "\nreturn 0; }\n"
    )
    import tempfile

    with tempfile.TemporaryDirectory() as tmp:
        src = f"{tmp}/layout.c"
        exe = f"{tmp}/layout"
        with open(src, "w") as f:
            f.write(source)
        subprocess.run(["gcc", "-std=c99", f"-I{ROOT / 'include'}", src, "-o", exe], check=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout
    return {k: int(v) for k, v in (line.split() for line in out.splitlines())}


@pytest.mark.parametrize("name", ["FwdParams", "DecodeParams", "AppendParams", "FsmnParams", "PagedKV", "LocalParams"])
def test_ctypes_structs_match_c_layout(name):
    from asrback_amd import _lib

    cls = getattr(_lib, name)
    struct = {"FwdParams": "asrattn_fwd_params", "DecodeParams": "asrattn_decode_params",
              "AppendParams": "asrattn_append_params", "FsmnParams": "asrattn_fsmn_params",
              "PagedKV": "asrattn_paged_kv", "LocalParams": "asrattn_local_params"}[name]
    fields = [f for f, _ in cls._fields_]
    layout = _c_layout(struct, fields)
    assert layout.pop("sizeof") == ctypes.sizeof(cls)
    for field in fields:
        assert layout[field] == getattr(cls, field).offset, field


def test_invalid_arguments_are_reported_not_fatal(lib):
    from asrback_amd import _lib

    p = _lib.DecodeParams()
    p.batch, p.heads_q, p.heads_kv, p.head_dim, p.max_len_k = 1, 3, 2, 64, 10
    p.dtype, p.scale = _lib.BF16, 0.125
    status = lib.asrattn_decode(ctypes.byref(p), None, 0, None)
    assert status == _lib.ERR_INVALID
    assert b"heads_q" in lib.asrattn_last_error()

    p.heads_q, p.heads_kv, p.head_dim = 2, 2, 96
    assert lib.asrattn_decode(ctypes.byref(p), None, 0, None) == _lib.ERR_UNSUPPORTED
    assert lib.asrattn_decode_workspace_size(ctypes.byref(p)) == ctypes.c_size_t(-1).value

    f = _lib.FwdParams()
    f.batch, f.heads_q, f.heads_kv, f.head_dim = 1, 1, 1, 64
    f.max_len_q = f.max_len_k = 4
    f.dtype, f.scale, f.causal = _lib.F32, 0.125, 7
    assert lib.asrattn_fwd(ctypes.byref(f), None) == _lib.ERR_INVALID
    assert b"causal" in lib.asrattn_last_error()
    f.causal, f.scale = 0, float("nan")
    assert lib.asrattn_fwd(ctypes.byref(f), None) == _lib.ERR_INVALID
    f.scale = 0.125  # valid shape but NULL tensors
    assert lib.asrattn_fwd(ctypes.byref(f), None) == _lib.ERR_INVALID
    assert b"non-NULL" in lib.asrattn_last_error()


def test_noalloc_rejects_partials_beyond_its_scratch(lib):
    """asrattn_decode_noalloc refuses split partials larger than its static
    array before any device call (stand-in pointers, never dereferenced)."""
    from asrback_amd import _lib

    p = _lib.DecodeParams()
    p.batch, p.heads_q, p.heads_kv, p.head_dim, p.max_len_k = 1, 8, 1, 256, 1 << 16
    p.dtype, p.scale = _lib.BF16, 0.0625
    p.q = p.k = p.v = p.out = 4096
    p.q_batch_stride, p.q_head_stride = 2048, 256
    p.k_batch_stride, p.k_token_stride, p.k_head_stride = 256 << 16, 256, 256
    p.v_batch_stride, p.v_token_stride, p.v_head_stride = 256 << 16, 256, 256
    p.o_batch_stride, p.o_head_stride = 2048, 256
    p.num_splits = 1024  # 8 rows x 1024 splits x 256 floats = 8 MiB of partials, plus their stats
    assert lib.asrattn_decode_workspace_size(ctypes.byref(p)) > 8 << 20
    assert lib.asrattn_decode_noalloc(ctypes.byref(p), None) == _lib.ERR_WORKSPACE
    assert b"scratch" in lib.asrattn_last_error()
    p.heads_q = 0  # argument errors come first, as in asrattn_decode
    assert lib.asrattn_decode_noalloc(ctypes.byref(p), None) == _lib.ERR_INVALID


def test_invalid_append_and_span_are_reported(lib):
    """Every check below fails before any device call (the pointers are
    stand-ins, never dereferenced)."""
    from asrback_amd import _lib

    p = _lib.DecodeParams()
    p.batch, p.heads_q, p.heads_kv, p.head_dim, p.max_len_k = 2, 4, 2, 128, 64
    p.dtype, p.scale = _lib.BF16, 0.125
    p.q = p.k = p.v = p.out = 4096
    p.q_batch_stride, p.q_head_stride = 512, 128
    p.k_batch_stride, p.k_token_stride, p.k_head_stride = 64 * 256, 256, 128
    p.v_batch_stride, p.v_token_stride, p.v_head_stride = 64 * 256, 256, 128
    p.o_batch_stride, p.o_head_stride = 512, 128
    a = _lib.AppendParams()
    assert lib.asrattn_decode_append(ctypes.byref(p), None, None, 0, None) == _lib.ERR_INVALID
    assert lib.asrattn_decode_append(ctypes.byref(p), ctypes.byref(a), None, 0, None) == _lib.ERR_INVALID
    assert b"positions" in lib.asrattn_last_error()
    p.positions = 8192
    assert lib.asrattn_decode_append(ctypes.byref(p), ctypes.byref(a), None, 0, None) == _lib.ERR_INVALID
    assert b"k_new" in lib.asrattn_last_error()
    a.k_new = a.v_new = 4096
    a.kn_batch_stride = a.vn_batch_stride = 256
    a.kn_head_stride = a.vn_head_stride = 128
    a.q_norm = 4096  # without k_norm
    assert lib.asrattn_decode_append(ctypes.byref(p), ctypes.byref(a), None, 0, None) == _lib.ERR_INVALID
    assert b"pairs" in lib.asrattn_last_error()
    a.k_norm, a.eps = 4096, float("nan")
    assert lib.asrattn_decode_append(ctypes.byref(p), ctypes.byref(a), None, 0, None) == _lib.ERR_INVALID
    assert b"eps" in lib.asrattn_last_error()
    a.eps, a.cos, a.sin, a.rope_batch_stride = 1e-6, 4096, 4104, 128  # sin misaligned
    assert lib.asrattn_decode_append(ctypes.byref(p), ctypes.byref(a), None, 0, None) == _lib.ERR_INVALID
    assert b"16-byte" in lib.asrattn_last_error()
    # A sequence's keys spanning 2 GiB cannot be addressed with 32-bit offsets.
    p.positions, p.max_len_k = 0, 1 << 23
    assert lib.asrattn_decode(ctypes.byref(p), None, 0, None) == _lib.ERR_UNSUPPORTED
    assert b"2 GiB" in lib.asrattn_last_error()


def test_invalid_fsmn_arguments_are_reported(lib):
    """asrattn_fwd_fsmn's own checks, before any device call (stand-in
    pointers, never dereferenced)."""
    from asrback_amd import _lib

    f = _lib.FwdParams()
    f.batch, f.heads_q, f.heads_kv, f.head_dim = 2, 4, 4, 128
    f.max_len_q = f.max_len_k = 40
    f.dtype, f.scale = _lib.BF16, 0.125
    f.q, f.k, f.v, f.out = 4096, 4096 + 1024, 4096 + 2048, 1 << 20
    for prefix in ("q", "k", "v"):
        setattr(f, f"{prefix}_batch_stride", 40 * 1536)
        setattr(f, f"{prefix}_token_stride", 1536)
        setattr(f, f"{prefix}_head_stride", 128)
    f.o_batch_stride, f.o_token_stride, f.o_head_stride = 40 * 512, 512, 128
    m = _lib.FsmnParams()
    assert lib.asrattn_fwd_fsmn(ctypes.byref(f), None, None) == _lib.ERR_INVALID
    assert lib.asrattn_fwd_fsmn(ctypes.byref(f), ctypes.byref(m), None) == _lib.ERR_UNSUPPORTED
    assert b"kernel_size" in lib.asrattn_last_error()
    m.kernel_size = 11
    assert lib.asrattn_fwd_fsmn(ctypes.byref(f), ctypes.byref(m), None) == _lib.ERR_INVALID
    assert b"non-NULL" in lib.asrattn_last_error()
    m.weight, m.memory, m.m_batch_stride, m.m_token_stride = 8192, 4100, 40 * 512, 512  # memory misaligned
    assert lib.asrattn_fwd_fsmn(ctypes.byref(f), ctypes.byref(m), None) == _lib.ERR_INVALID
    assert b"16-byte" in lib.asrattn_last_error()
    m.memory = 1 << 24
    f.causal = _lib.CAUSAL_TOP_LEFT
    assert lib.asrattn_fwd_fsmn(ctypes.byref(f), ctypes.byref(m), None) == _lib.ERR_INVALID
    assert b"non-causal" in lib.asrattn_last_error()
    f.causal, f.heads_kv = _lib.CAUSAL_NONE, 2
    assert lib.asrattn_fwd_fsmn(ctypes.byref(f), ctypes.byref(m), None) == _lib.ERR_INVALID
    f.heads_kv, f.max_len_k = 4, 39
    assert lib.asrattn_fwd_fsmn(ctypes.byref(f), ctypes.byref(m), None) == _lib.ERR_INVALID
    f.max_len_k, m.kernel_size = 40, 16
    assert lib.asrattn_fwd_fsmn(ctypes.byref(f), ctypes.byref(m), None) == _lib.ERR_UNSUPPORTED
    # Nothing to do: no device call, no error.
    m.kernel_size, f.batch = 11, 0
    assert lib.asrattn_fwd_fsmn(ctypes.byref(f), ctypes.byref(m), None) == _lib.OK


def test_invalid_paged_arguments_are_reported(lib):
    """asrattn_decode_paged's checks, before any device call (stand-in
    pointers, never dereferenced)."""
    from asrback_amd import _lib

    p = _lib.DecodeParams()
    p.batch, p.heads_q, p.heads_kv, p.head_dim, p.max_len_k = 2, 4, 2, 128, 1024
    p.dtype, p.scale = _lib.BF16, 0.125
    p.q = p.k = p.v = p.out = 4096
    p.q_batch_stride, p.q_head_stride = 512, 128
    p.k_token_stride, p.k_head_stride = 256, 128
    p.v_token_stride, p.v_head_stride = 256, 128
    p.o_batch_stride, p.o_head_stride = 512, 128
    pk = _lib.PagedKV()
    assert lib.asrattn_decode_paged(ctypes.byref(p), None, None, None, 0, None) == _lib.ERR_INVALID
    assert lib.asrattn_decode_paged(ctypes.byref(p), None, ctypes.byref(pk), None, 0, None) == _lib.ERR_INVALID
    assert b"block_table" in lib.asrattn_last_error()
    pk.block_table, pk.bt_stride, pk.num_pages = 8192, 16, 100
    pk.k_page_stride = pk.v_page_stride = 64 * 256
    for bad in (0, 8, 48):  # not a power of two >= 16
        pk.page_size = bad
        assert lib.asrattn_decode_paged(ctypes.byref(p), None, ctypes.byref(pk), None, 0, None) == _lib.ERR_UNSUPPORTED
        assert b"page_size" in lib.asrattn_last_error()
    pk.page_size = 32  # 16 pages of 32 cannot reach 1024 keys
    assert lib.asrattn_decode_paged(ctypes.byref(p), None, ctypes.byref(pk), None, 0, None) == _lib.ERR_INVALID
    assert b"reach" in lib.asrattn_last_error()
    pk.page_size, pk.k_page_stride = 64, 64 * 256 + 4  # page stride not a multiple of 16 bytes
    assert lib.asrattn_decode_paged(ctypes.byref(p), None, ctypes.byref(pk), None, 0, None) == _lib.ERR_INVALID
    assert b"page strides" in lib.asrattn_last_error()
    # bf16 at head_dim 64: a wave covers 8 keys per load, so pages hold >= 32.
    p.head_dim, p.q_head_stride, p.k_head_stride, p.v_head_stride = 64, 64, 64, 64
    pk.k_page_stride, pk.page_size, pk.bt_stride = 64 * 256, 16, 64
    assert lib.asrattn_decode_paged(ctypes.byref(p), None, ctypes.byref(pk), None, 0, None) == _lib.ERR_UNSUPPORTED
    assert b">= 32" in lib.asrattn_last_error()


def test_invalid_window_and_local_arguments_are_reported(lib):
    """Window and blocked-local-attention checks, before any device call."""
    from asrback_amd import _lib

    f = _lib.FwdParams()
    f.batch, f.heads_q, f.heads_kv, f.head_dim = 1, 8, 1, 256
    f.max_len_q = f.max_len_k = 4
    f.dtype, f.scale, f.window = _lib.BF16, 1.0, 512
    assert lib.asrattn_fwd(ctypes.byref(f), None) == _lib.ERR_INVALID  # a window needs causal attention
    assert b"window" in lib.asrattn_last_error()
    f.causal, f.window = _lib.CAUSAL_TOP_LEFT, -1
    assert lib.asrattn_fwd(ctypes.byref(f), None) == _lib.ERR_INVALID
    d = _lib.DecodeParams()
    d.batch, d.heads_q, d.heads_kv, d.head_dim, d.max_len_k = 1, 8, 1, 512, 16
    d.dtype, d.scale, d.window = _lib.F32, 1.0, 0
    assert lib.asrattn_decode(ctypes.byref(d), None, 0, None) == _lib.ERR_UNSUPPORTED  # fp32 at 512
    d.dtype, d.window = _lib.BF16, -3
    assert lib.asrattn_decode(ctypes.byref(d), None, 0, None) == _lib.ERR_INVALID
    p = _lib.LocalParams()
    p.batch, p.tokens, p.heads, p.head_dim = 1, 10, 2, 64
    p.chunk, p.past, p.future, p.rel_positions, p.softcap, p.invalid = 12, 12, 0, 15, 50.0, -1e9
    assert lib.asrattn_local(ctypes.byref(p), None) == _lib.ERR_INVALID  # 15 > past + future + 2
    p.rel_positions, p.softcap = 13, 0.0
    assert lib.asrattn_local(ctypes.byref(p), None) == _lib.ERR_INVALID
    p.softcap, p.head_dim = 50.0, 1024  # the block's staging exceeds 64 KB of LDS
    assert lib.asrattn_local(ctypes.byref(p), None) == _lib.ERR_UNSUPPORTED
    p.head_dim = 64
    assert lib.asrattn_local(ctypes.byref(p), None) == _lib.ERR_INVALID  # NULL tensors
    assert b"non-NULL" in lib.asrattn_last_error()


def test_workspace_size_and_split_choice(lib):
    from asrback_amd import _lib

    p = _lib.DecodeParams()
    # Whisper-small cross-attention: 16 rows x 12 heads over 1500 frames is
    # enough (sequence, head) pairs for one split; whisper-tiny's batch of one
    # (6 heads) splits its keys.
    p.batch, p.heads_q, p.heads_kv, p.head_dim, p.max_len_k = 16, 12, 12, 64, 1500
    p.dtype, p.scale = _lib.BF16, 0.125
    assert lib.asrattn_decode_num_splits(ctypes.byref(p)) == 1
    assert lib.asrattn_decode_workspace_size(ctypes.byref(p)) == 0
    # Gemma 4's 32 rows x 4 kv heads (128 pairs) take two splits.
    p.batch, p.heads_q, p.heads_kv, p.head_dim, p.max_len_k = 32, 8, 4, 256, 1280
    assert lib.asrattn_decode_num_splits(ctypes.byref(p)) == 2
    p.head_dim, p.max_len_k = 64, 1500
    p.batch, p.heads_q, p.heads_kv = 1, 6, 6
    splits = lib.asrattn_decode_num_splits(ctypes.byref(p))
    assert splits == 6  # 1500 keys, at least 256 per split

    def up(n):
        return (n + 255) // 256 * 256

    rows = 6 * splits
    assert lib.asrattn_decode_workspace_size(ctypes.byref(p)) == up(rows * 64 * 4) + up(rows * 8)
    p.num_splits = 1
    assert lib.asrattn_decode_workspace_size(ctypes.byref(p)) == 0
    assert lib.asrattn_decode_num_splits(ctypes.byref(p)) == 1
    # A missing workspace is an error, not a fault.
    p.num_splits = 4
    p.q = p.k = p.v = p.out = 16
    assert lib.asrattn_decode(ctypes.byref(p), None, 0, None) == _lib.ERR_WORKSPACE


def test_choose_workspace_size_and_errors(lib):
    """Qwen3's (64, 151936) logits split each row over 32 workgroups
    (one 16-byte partial each); small vocabularies need no workspace; a
    short workspace is an error, not a fault."""
    from asrback_amd import _lib

    assert lib.asrattn_choose_workspace_size(64, 151936) == 64 * 32 * 16
    assert lib.asrattn_choose_workspace_size(4, 2000) == 0
    assert lib.asrattn_choose_workspace_size(0, 151936) == 0
    fake = 64  # never dereferenced: the checks come first
    status = lib.asrattn_choose(fake, 64, 151936, 151936, None, fake, fake, fake, 16, None)
    assert status == _lib.ERR_WORKSPACE
    assert b"workspace" in lib.asrattn_last_error()
    assert lib.asrattn_choose(fake, 64, 151936, 151936, None, fake, fake, None, 16, None) == _lib.ERR_INVALID


def test_zero_padded_rows_needs_the_padded_noncausal_layout(lib):
    """ASRATTN_FWD_ZERO_PADDED_ROWS is refused with cu_seqlens, with causal
    attention and without seqused_k, before any device call (the pointers
    are stand-ins, never dereferenced)."""
    from asrback_amd import _lib

    def params():
        f = _lib.FwdParams()
        f.batch, f.heads_q, f.heads_kv, f.head_dim = 2, 4, 4, 128
        f.max_len_q = f.max_len_k = 300
        f.dtype, f.scale, f.flags = _lib.BF16, 128**-0.5, 2  # ASRATTN_FWD_ZERO_PADDED_ROWS
        f.q = f.k = f.v = f.out = 4096
        f.seqused_k = 64
        return f

    f = params()
    f.cu_seqlens_q = f.cu_seqlens_k = 128
    assert lib.asrattn_fwd(ctypes.byref(f), None) == _lib.ERR_INVALID
    assert b"ZERO_PADDED_ROWS" in lib.asrattn_last_error()
    f = params()
    f.causal = 1
    assert lib.asrattn_fwd(ctypes.byref(f), None) == _lib.ERR_INVALID
    assert b"ZERO_PADDED_ROWS" in lib.asrattn_last_error()
    f = params()
    f.seqused_k = None
    assert lib.asrattn_fwd(ctypes.byref(f), None) == _lib.ERR_INVALID
    assert b"ZERO_PADDED_ROWS" in lib.asrattn_last_error()
