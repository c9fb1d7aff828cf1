"""The C ABI library loads, exports every function ``include/*.h`` declares, its ctypes mirrors match
the C struct layouts, and argument errors come back as status codes without touching a GPU."""
import ctypes
import glob
import os
import re
import subprocess
import tempfile

import pytest

from worldattention_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))


def declared_functions():
    names = []
    for h in HEADERS:
        text = open(h).read()
        names += re.findall(r"^\s*(?:int|int64_t|const char\s*\*)\s+(wa_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def declared_structs():
    names = []
    for h in HEADERS:
        names += re.findall(r"typedef struct (wa_\w+)\s*\{", open(h).read())
    return names


def test_library_loads_and_reports_version():
    assert os.path.exists(_lib.LIB_PATH), "run __graft_entry__.build() first"
    assert _lib.lib().wa_version() >= 100


def test_every_declared_function_is_exported_and_bound():
    funcs = declared_functions()
    assert len(funcs) >= 10
    handle = ctypes.CDLL(_lib.LIB_PATH)
    for name in funcs:
        assert hasattr(handle, name), f"{name} declared but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"


def test_ctypes_structs_match_the_c_layout():
    structs = declared_structs()
    mirrors = {cls._name: cls for cls in (getattr(_lib, n) for n in dir(_lib))
               if isinstance(cls, type) and issubclass(cls, ctypes.Structure)
               for cls._name in [cls.__name__]}
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADERS[0]}"', "int main(void) {"]
    for s in structs:
        lines.append(f'  printf("{s} size %zu\\n", sizeof({s}));')
        for field, _ in mirrors[s]._fields_:
            lines.append(f'  printf("{s} {field} %zu\\n", offsetof({s}, {field}));')
    lines.append("  return 0; }")
    with tempfile.TemporaryDirectory() as tmp:
        src, exe = os.path.join(tmp, "layout.c"), os.path.join(tmp, "layout")
        open(src, "w").write("\n".join(lines))
        subprocess.run(["gcc", "-o", exe, src], check=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout.split("\n")
    for line in filter(None, out):
        s, field, val = line.split()
        cls = mirrors[s]
        if field == "size":
            assert ctypes.sizeof(cls) == int(val), f"{s} size"
        else:
            assert getattr(cls, field).offset == int(val), f"{s}.{field}"


def test_argument_errors_return_status_without_a_gpu():
    handle = _lib.lib()
    assert handle.wa_bsa_fwd(None, None) == -1
    assert b"null" in handle.wa_last_error()
    args = _lib.BsaFwdArgs()
    args.D, args.block_size = 96, 64
    assert handle.wa_bsa_fwd(ctypes.byref(args), None) == -1
    assert b"head dim" in handle.wa_last_error()
    rargs = _lib.RouteArgs()
    rargs.index = rargs.num = 16
    rargs.probs = 16
    rargs.Nkv, rargs.H = 5000, 1
    assert handle.wa_route(ctypes.byref(rargs), None) == -1
    assert handle.wa_map_to_index(None, 1, 1, None, None, None) == -1
    assert handle.wa_route_workspace_bytes(1, 12, 37, 256) >= 12 * 37 * 257 * 4


def test_noalloc_rejects_oversized_launches_and_workspaces_without_a_gpu():
    """wa_bsa_fwd_noalloc refuses, on the host and before any HIP call, a launch whose workspace
    would not fit the static array and a caller-supplied workspace. The tensor pointers are dummy
    aligned addresses and there is no stream: nothing is dereferenced or launched."""
    handle = _lib.lib()
    fake = 1 << 20
    h, d, length = 64, 128, 40000
    args = _lib.BsaFwdArgs()
    args.q = args.k = args.v = args.o = args.index = args.num = fake
    for name in ("q", "k", "v", "o"):
        setattr(args, name + "_sb", length * h * d)
        setattr(args, name + "_st", h * d)
        setattr(args, name + "_sh", d)
    args.o_dtype = _lib.WA_BF16
    args.index_width = 64
    args.B, args.H, args.Lq, args.Lkv, args.D, args.block_size = 1, h, length, length, d, 128
    args.max_visits, args.split_visits = 64, 16
    # 64 heads x 313 query blocks x 4 split units of partials: far beyond the static array
    need = handle.wa_bsa_fwd_workspace_bytes(h * 313, 64, 16, 128, d)
    assert need > _lib.BSA_FWD_NOALLOC_SCRATCH_BYTES
    assert handle.wa_bsa_fwd_noalloc(ctypes.byref(args), None) == _lib.WA_ERR_ARG
    assert b"static scratch" in handle.wa_last_error()
    args.workspace = fake
    assert handle.wa_bsa_fwd_noalloc(ctypes.byref(args), None) == _lib.WA_ERR_ARG
    assert b"must be NULL" in handle.wa_last_error()


def test_one_call_entry_points_reject_bad_arguments_without_a_gpu():
    """wa_hsa_fwd / wa_hsa_bwd argument checks run on the host before any HIP call: dummy aligned
    pointers, no stream, nothing dereferenced or launched."""
    handle = _lib.lib()
    fake = 1 << 20
    assert handle.wa_hsa_bwd(None, None) == _lib.WA_ERR_ARG
    b = _lib.HsaBwdArgs()
    b.q = b.k = b.v = b.dout = b.dq = b.dk = b.dv = b.workspace = fake
    b.B, b.H, b.Lq, b.Lkv, b.D, b.block_size = 1, 4, 256, 512, 128, 128
    b.n_sparse, b.n_linear = 2, 2
    b.block_size = 96
    assert handle.wa_hsa_bwd(ctypes.byref(b), None) == _lib.WA_ERR_ARG
    assert b"block size" in handle.wa_last_error()
    b.block_size = 128
    assert handle.wa_hsa_bwd(ctypes.byref(b), None) == _lib.WA_ERR_ARG  # sparse heads without routing
    assert b"sparse heads need" in handle.wa_last_error()
    b.sparse_heads = b.index = b.num = b.lse = b.o = fake
    assert handle.wa_hsa_bwd(ctypes.byref(b), None) == _lib.WA_ERR_ARG  # linear heads without their state
    assert b"linear heads need" in handle.wa_last_error()
    b.linear_heads = b.lin_modes = b.lin = b.gate = b.state = b.zsum = fake
    b.gate_w = fake
    assert handle.wa_hsa_bwd(ctypes.byref(b), None) == _lib.WA_ERR_ARG  # gate weight without its gradients
    assert b"dgate_w" in handle.wa_last_error()
    b.dgate_w = b.dgate_b = fake
    b.side_stream = fake
    assert handle.wa_hsa_bwd(ctypes.byref(b), None) == _lib.WA_ERR_ARG  # side stream without events
    assert b"fork and join" in handle.wa_last_error()
    b.side_stream = None
    b.dq_stream = fake
    assert handle.wa_hsa_bwd(ctypes.byref(b), None) == _lib.WA_ERR_ARG
    assert b"dQ stream" in handle.wa_last_error()
    b.dq_stream = None
    b.dq_dtype, b.dq_sb = _lib.WA_BF16, 3   # a bf16 dq with a stride that breaks 16-byte rows
    assert handle.wa_hsa_bwd(ctypes.byref(b), None) == _lib.WA_ERR_ARG
    assert b"bf16 dq" in handle.wa_last_error()
    assert handle.wa_hsa_bwd_workspace_bytes(1, 12, 4680, 32760, 128, 128, 8, 4) > 0

    f = _lib.HsaFwdArgs()
    f.q = f.k = f.v = f.o = f.workspace = fake
    f.B, f.H, f.Lq, f.Lkv, f.D, f.block_size = 1, 4, 256, 512, 128, 128
    f.linear_heads, f.n_linear = fake, 2
    f.lin = fake                             # an unfused readout without its gate and modes
    assert handle.wa_hsa_fwd(ctypes.byref(f), None) == _lib.WA_ERR_ARG
    assert b"lin_modes" in handle.wa_last_error()
    f.gate = f.lin_modes = fake
    f.state = fake                           # state without zsum
    assert handle.wa_hsa_fwd(ctypes.byref(f), None) == _lib.WA_ERR_ARG
    assert b"state and zsum" in handle.wa_last_error()
