"""C-ABI boundary checks that run without a GPU.

* ``libtops_gla.so`` loads and exports every function ``include/tops_gla.h`` declares, with
  the argument count the Python binding uses.
* Invalid arguments are rejected by the host-side validator with the documented status code
  and message, before any HIP call (so these calls are safe on a machine without a GPU).
* The Python API refuses CPU tensors (there is no CPU fallback).
"""

import ctypes
import os
import re

import pytest
import torch

from tops import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tops_gla.h")


def _declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(?:int|int64_t|float|const char\*)\s+(tops_gla_\w+)\s*\(([^)]*)\)\s*;", src):
        params = [p for p in m.group(2).split(",") if p.strip() and p.strip() != "void"]
        out[m.group(1)] = len(params)
    return out


def test_header_lists_entry_points():
    decl = _declared()
    assert len(decl) == 32, decl
    assert set(decl) == set(_lib.EXPORTED)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name, nargs in _declared().items():
        assert hasattr(lib, name), f"{name} not exported"
        if name in _lib._SIGS:
            assert len(_lib._SIGS[name]) == nargs, f"{name}: binding has {len(_lib._SIGS[name])}"\
                f" args, header declares {nargs}"
    assert lib.tops_gla_version().startswith(b"tops-gla-mi355x")


def _rc(name, *args):
    lib = _lib.load()
    rc = getattr(lib, name)(*args)
    return rc, lib.tops_gla_last_error().decode()


NULL = None


def test_chunk_fwd_rejects_bad_dtype():
    rc, msg = _rc("tops_gla_chunk_fwd", NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL,
                  0, 1.0, 1, 64, 1, 64, 64, 64, NULL, NULL, 1, 1, 7, NULL)
    assert rc == 1 and "dtype" in msg


def test_chunk_fwd_rejects_unsupported_chunk():
    rc, msg = _rc("tops_gla_chunk_fwd", NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL,
                  0, 1.0, 1, 64, 1, 64, 64, 48, NULL, NULL, 1, 2, 1, NULL)
    assert rc == 2 and "chunk_size" in msg


def test_chunk_fwd_rejects_wrong_chunk_count():
    rc, msg = _rc("tops_gla_chunk_fwd", NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL,
                  0, 1.0, 2, 100, 1, 64, 64, 64, NULL, NULL, 2, 3, 1, NULL)
    assert rc == 1 and "NC" in msg


def test_chunk_fwd_rejects_null_buffers():
    rc, msg = _rc("tops_gla_chunk_fwd", NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL,
                  0, 1.0, 1, 64, 1, 64, 64, 64, NULL, NULL, 1, 1, 1, NULL)
    assert rc == 1 and "NULL" in msg


def test_varlen_requires_batch_one():
    fake = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    rc, msg = _rc("tops_gla_chunk_fwd_h", fake, fake, fake, 0, NULL, NULL, NULL, NULL, 0, 2, 64,
                  1, 64,
                  64, 64, fake, fake, 2, 2, 1, NULL)
    assert rc == 1 and "B == 1" in msg


def test_lds_budget_reported():
    rc, msg = _rc("tops_gla_chunk_fwd_o", NULL, NULL, NULL, NULL, 0, NULL, NULL, NULL, NULL,
                  1.0, 1, 64, 1, 2048, 64, 64, NULL, NULL, 1, 1, 0, NULL)
    assert rc == 2 and "LDS" in msg


def test_small_chunks_validated_on_the_host():
    """Chunk sizes 4 and 8 reach the small-chunk kernels' own checks (K limit, NULL inputs)."""
    for C in (4, 8):
        rc, msg = _rc("tops_gla_chunk_fwd_o", NULL, NULL, NULL, NULL, 0, NULL, NULL, NULL, NULL,
                      1.0, 1, 64, 1, 4096, 64, C, NULL, NULL, 1, 64 // C, 0, NULL)
        assert rc == 2 and "K=4096" in msg, msg
        rc, msg = _rc("tops_gla_chunk_fwd_h", NULL, NULL, NULL, 0, NULL, NULL, NULL, NULL, 0, 1,
                      64, 1, 64, 64, C, NULL, NULL, 1, 64 // C, 1, NULL)
        assert rc == 1 and "NULL" in msg, msg
        rc, msg = _rc("tops_gla_chunk_bwd_dh", NULL, NULL, 0, NULL, NULL, NULL, NULL, NULL, 0,
                      1.0, 1, 64, 1, 64, 64, C, NULL, NULL, 1, 64 // C + 1, 1, NULL)
        assert rc == 1 and "NC" in msg, msg


def test_recurrent_rejects_large_k():
    rc, msg = _rc("tops_gla_fused_recurrent_fwd", NULL, NULL, NULL, NULL, NULL, NULL, NULL,
                  NULL, 1.0, 0, 1, 8, 1, 1024, 64, NULL, 1, 1, 0, NULL)
    assert rc == 2 and "K <= 512" in msg


def test_recurrent_bwd_validation():
    args = lambda **kw: [kw.get(n, NULL) for n in (  # noqa: E731
        "q", "k", "v", "gk", "gv", "o", "do", "dht", "h0", "dq", "dk", "dv", "dgk", "dgv",
        "dh0", "ht")]
    tail = lambda K, V: [1.0, 0, 1, 8, 1, K, V, NULL, 1, 1, NULL]  # noqa: E731
    rc, msg = _rc("tops_gla_fused_recurrent_bwd", *args(), *tail(1024, 64))
    assert rc == 2 and "K, V <= 512" in msg
    buf = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    full = dict(q=buf, k=buf, v=buf, do=buf, dq=buf, dk=buf, dv=buf)
    rc, msg = _rc("tops_gla_fused_recurrent_bwd", *args(**full, gk=buf), *tail(64, 64))
    assert rc == 1 and "dgk must be given" in msg
    rc, msg = _rc("tops_gla_fused_recurrent_bwd", *args(**full, gv=buf, dgv=buf), *tail(64, 64))
    assert rc == 1 and "o (forward output) is required" in msg
    rc, msg = _rc("tops_gla_fused_recurrent_bwd", *args(**full, gk=buf, dgk=buf, dht=buf),
                  *tail(64, 64))
    assert rc == 1 and "ht_ws is required" in msg
    rc, msg = _rc("tops_gla_fused_recurrent_bwd", *args(q=buf), *tail(64, 64))
    assert rc == 1 and "must not be NULL" in msg


def test_cumsum_rejects_non_power_of_two():
    rc, msg = _rc("tops_gla_chunk_local_cumsum", NULL, NULL, 1, 8, 1, 4, 12, 0, 0, 1.0, 0,
                  NULL, NULL, 1, 1, 0, 0, NULL)
    assert rc == 1 and "power of 2" in msg


def test_empty_problem_is_a_no_op():
    # zero tokens: valid, nothing launched (safe without a GPU)
    rc, msg = _rc("tops_gla_chunk_local_cumsum", NULL, NULL, 1, 0, 1, 4, 16, 0, 0, 1.0, 0, NULL,
                  NULL, 1, 0, 0, 0, NULL)
    assert rc == 0 and msg == ""


def test_python_api_refuses_cpu_tensors():
    from tops.ops.gla import chunk_gla, fused_recurrent_gla

    q = torch.randn(1, 16, 1, 8)
    v = torch.randn(1, 16, 1, 8)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        chunk_gla(q, q, v, torch.zeros_like(q))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        fused_recurrent_gla(q, q, v, gk=torch.zeros_like(q))


def test_python_api_asserts_shapes_like_reference():
    from tops.ops.gla import fused_recurrent_gla

    q = torch.randn(1, 16, 2, 8)
    with pytest.raises(AssertionError, match="Expected k shape"):
        fused_recurrent_gla(q, q[:, :, :1], q)


def test_seq_layout_chunk_offsets():
    s = _lib.SeqLayout(1, 50, 16, [0, 13, 37, 50], "cpu")
    assert (s.N, s.NC) == (3, 1 + 2 + 1)
    assert s.chunk_cu.tolist() == [0, 1, 3, 4]
    f = _lib.SeqLayout(3, 37, 16, None, "cpu")
    assert (f.N, f.NC) == (3, 9) and f.cu is None


def test_segment_workspace_query():
    """Host-only: the workspace = segment states [N, NS, H, K, V] f32 + decays (full-head
    kernels), the gate-range flags (int32: per chunk and head, or per full-head block where
    that is more), the wide heads' gating, and for the backward the fallback's final states
    [N, H, K, V] f32; each part 256-byte aligned."""
    lib = _lib.load()
    q = lib.tops_gla_chunk_ws_bytes
    a = lambda x: (x + 255) // 256 * 256  # noqa: E731
    # B4 T8192 H16 K=V=128 chunk 64 bf16: 128 chunks per sequence; 64 (sequence, head) blocks
    # -> 4 segments of 32 chunks (one block per CU of 256)
    st = 4 * 4 * 16 * 128 * 128 * 4
    gm = 4 * 4 * 16 * 128 * 4
    flags = a(4 * 128 * 16 * 4)          # per chunk and head (more than the 256 blocks)
    ht = 4 * 16 * 128 * 128 * 4
    assert q(4, 8192, 16, 128, 128, 64, 4, 0, 1, 1) == a(st + a(gm)) + flags + ht
    assert q(4, 8192, 16, 128, 128, 64, 4, 0, 1, 0) == a(st + a(gm)) + flags   # forward
    # varlen (3 sequences): unsegmented; flags for at most 8192 / 64 + 3 chunks per head
    assert q(1, 8192, 16, 128, 128, 64, 3, 1, 1, 1) == a(131 * 16 * 4) + 3 * 16 * 128 * 128 * 4
    assert q(4, 8192, 16, 128, 128, 64, 3, 0, 1, 1) == 0    # fixed length needs N == B
    # float32 and chunk 32 (the per-chunk kernels): flags and fallback states only
    assert q(4, 8192, 16, 128, 128, 64, 4, 0, 0, 1) == flags + ht
    assert q(4, 8192, 16, 128, 128, 32, 4, 0, 1, 1) == a(4 * 256 * 16 * 4) + ht
    assert q(4, 8192, 16, 128, 128, 32, 4, 0, 1, 0) == a(4 * 256 * 16 * 4)
    # 4 chunks: too short to split; flags and fallback states
    assert q(1, 256, 2, 64, 64, 64, 1, 0, 1, 1) == a(4 * 2 * 4) + 2 * 64 * 64 * 4
    # K = 256: V tiles of 64 columns (2 per head) -> 2 segments of 64 chunks; the fallback's
    # states for the per-chunk backward
    st2, gm2 = 4 * 2 * 16 * 256 * 128 * 4, 4 * 2 * 16 * 256 * 4
    assert q(4, 8192, 16, 256, 128, 64, 4, 0, 1, 1) == (a(st2 + a(gm2)) + flags
                                                        + 4 * 16 * 256 * 128 * 4)
    # K = 320 (per-chunk kernels): flags and states; K or V past 512: no fallback states
    assert q(4, 8192, 16, 320, 128, 64, 4, 0, 1, 1) == flags + 4 * 16 * 320 * 128 * 4
    assert q(4, 8192, 16, 128, 640, 64, 4, 0, 1, 1) == flags
    assert q(4, 8192, 16, 640, 128, 64, 4, 0, 1, 1) == 0    # K > 512: nothing checked


def test_kernel_timer_without_launches():
    # host-only: with no timed launch recorded the timer reports -1 (no HIP call is made)
    lib = _lib.load()
    assert lib.tops_gla_kernel_ms(0) == -1.0
    assert lib.tops_gla_kernel_ms(1) == -1.0
    assert lib.tops_gla_kernel_ms(7) == -1.0


def test_simple_chunk_validation():
    buf = ctypes.c_void_p(256)  # never dereferenced: validation fails first
    fwd = lambda gs, ts, dtype, K=128: [buf, buf, buf, gs, ts, NULL, buf, NULL, NULL, NULL, 0,  # noqa: E731
                                        1.0, 1, 64, 2, K, 128, 64, NULL, NULL, 1, 1, dtype, NULL]
    rc, msg = _rc("tops_gla_simple_chunk_fwd", *fwd(NULL, 0, 1))
    assert rc == 1 and "gs must not be NULL" in msg
    rc, msg = _rc("tops_gla_simple_chunk_fwd", *fwd(buf, 3, 1))
    assert rc == 1 and "gs_ts must be 0 or H" in msg
    rc, msg = _rc("tops_gla_simple_chunk_fwd", *fwd(buf, 2, 0))   # float32: not full-head
    assert rc == 2 and "full-head" in msg
    bwd = lambda K, V: [buf, buf, buf, buf, 0, NULL, buf, buf, NULL, buf, buf, buf, NULL, NULL,  # noqa: E731
                        NULL, NULL, 0, 1.0, 1, 64, 2, K, V, 64, NULL, NULL, 1, 1, 1, NULL]
    rc, msg = _rc("tops_gla_simple_chunk_bwd", *bwd(128, 256))   # the fused backward: V <= 128
    assert rc == 2 and "full-head" in msg
    rc, msg = _rc("tops_gla_simple_chunk_bwd", *(bwd(128, 128)[:6] + [NULL] + bwd(128, 128)[7:]))
    assert rc == 1 and "h_ws is required" in msg


def test_seq_layout_refuses_bad_cu_seqlens():
    """cu_seqlens must start at 0, increase strictly (no empty sequence) and end within T;
    refused on the host, before anything reaches the device."""
    cpu = torch.device("cpu")
    for cu, msg in (([0, 3, 3, 10], "no empty sequences"), ([1, 5, 10], "strictly increasing"),
                    ([0, 6, 4, 10], "strictly increasing"), ([0, 4, 12], "exceeds T")):
        with pytest.raises(AssertionError, match=msg):
            _lib.SeqLayout(1, 10, 4, cu, cpu)


def test_argument_checks_survive_python_O():
    """The host checks that keep the kernels in bounds are raises, not asserts: they hold
    under ``python -O`` (which strips assert statements)."""
    import subprocess
    import sys

    code = (
        "import sys; sys.path[:0] = [%r]\n"
        "import torch\n"
        "from tops._lib import SeqLayout, ArgumentError\n"
        "import tops.ops.gla as G\n"
        "bad = [lambda: SeqLayout(1, 10, 64, [0, 5, 3], 'cpu'),\n"
        "       lambda: SeqLayout(1, 10, 64, [0, 5, 12], 'cpu'),\n"
        "       lambda: SeqLayout(2, 10, 64, [0, 5, 10], 'cpu'),\n"
        "       lambda: G.chunk_gla(torch.zeros(1, 8, 2, 16), torch.zeros(1, 8, 2, 8),\n"
        "                           torch.zeros(1, 8, 2, 16), torch.zeros(1, 8, 2, 16)),\n"
        "       lambda: G.fused_recurrent_gla(torch.zeros(1, 8, 2, 16), torch.zeros(1, 8, 2, 16),\n"
        "                                     torch.zeros(1, 7, 2, 16))]\n"
        "n = 0\n"
        "for f in bad:\n"
        "    try:\n"
        "        f()\n"
        "    except ArgumentError as e:\n"
        "        assert isinstance(e, ValueError) and isinstance(e, AssertionError)\n"
        "        n += 1\n"
        "print(n)\n" % os.path.join(ROOT, "pallas-kernel_amd"))
    out = subprocess.run([sys.executable, "-O", "-c", code], capture_output=True, text=True,
                         timeout=120)
    assert out.returncode == 0, out.stderr
    assert out.stdout.strip() == "5", out.stdout + out.stderr


def test_empty_sequences_are_left_out_on_the_host():
    from tops import _lib

    assert _lib.drop_empty([0, 3, 7]) == ([0, 3, 7], None)
    assert _lib.drop_empty([0, 0, 3, 3, 7, 7]) == ([0, 3, 7], [1, 3])
    assert _lib.drop_empty([0, 0]) == ([0], [])
    import torch

    h0 = torch.arange(4.0).reshape(4, 1)
    part = torch.tensor([[10.0], [30.0]])
    assert _lib.scatter_states(part, h0, [1, 3], (4, 1), "cpu").flatten().tolist() == \
        [0.0, 10.0, 2.0, 30.0]
    assert _lib.scatter_states(None, None, [], (2, 1), "cpu").flatten().tolist() == [0.0, 0.0]
    assert _lib.gather_states(h0, [1, 3]).flatten().tolist() == [1.0, 3.0]


def test_noalloc_forward_validates_on_the_host():
    """tops_gla_chunk_fwd_noalloc refuses bad arguments before touching the GPU (no scratch
    address is taken for them)."""
    rc, msg = _rc("tops_gla_chunk_fwd_noalloc", NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL,
                  1.0, 1, 64, 1, 64, 64, 64, NULL, NULL, 1, 1, 7, NULL)
    assert rc == 1 and "dtype" in msg
    rc, msg = _rc("tops_gla_chunk_fwd_noalloc", NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL,
                  1.0, 1, 64, 1, 64, 64, 64, NULL, NULL, 1, 1, 1, NULL)
    assert rc == 1 and "NULL" in msg


def test_concat_cols_rejects_bad_arguments():
    srcs = (ctypes.c_void_p * 2)(16, 32)
    rc, msg = _rc("tops_gla_concat_cols", srcs, (ctypes.c_int64 * 2)(1024, 3), 2, 0,
                  ctypes.c_void_p(64), 1, NULL)
    assert rc == 2 and "multiple of 16 bytes" in msg
    rc, msg = _rc("tops_gla_concat_cols", srcs, (ctypes.c_int64 * 2)(1024, 8), 9, 0,
                  ctypes.c_void_p(64), 1, NULL)
    assert rc == 1 and "nsrc" in msg
    rc, msg = _rc("tops_gla_concat_cols", srcs, (ctypes.c_int64 * 2)(1024, 8), 2, 0,
                  ctypes.c_void_p(64), 7, NULL)
    assert rc == 1 and "dtype" in msg
    # nothing to copy: accepted without a launch
    rc, _ = _rc("tops_gla_concat_cols", srcs, (ctypes.c_int64 * 2)(1024, 8), 2, 0,
                ctypes.c_void_p(64), 1, NULL)
    assert rc == 0
