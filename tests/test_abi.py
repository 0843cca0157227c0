"""The C ABI without a GPU: libelyhip.so loads, exports every function
include/ely.h declares (and nothing the Python binding expects is missing),
the header's constants match the binding's, and argument errors come back as
status codes and messages, never crashes.  No call here launches a kernel:
each one fails its argument check before touching the HIP runtime."""

from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "ely.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ely_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from elysium_wan_amd import _lib

    return _lib.load()


def test_library_exports_every_declared_function(lib):
    names = _declared()
    assert len(names) >= 15
    for n in names:
        assert hasattr(lib, n), n


def test_binding_covers_the_header():
    from elysium_wan_amd import _lib

    assert sorted(_lib.EXPORTS) == _declared()


def test_header_constants_match_the_binding():
    from elysium_wan_amd import _lib

    text = open(HEADER).read()
    consts = dict(re.findall(r"\b(ELY_\w+)\s*=\s*(\d+)", text))
    assert int(consts["ELY_F32"]) == _lib.F32 and int(consts["ELY_BF16"]) == _lib.BF16
    assert int(consts["ELY_E4M3"]) == _lib.E4M3 and int(consts["ELY_E5M2"]) == _lib.E5M2
    assert int(consts["ELY_ORDER_HOST"]) == _lib.ORDER_HOST and int(consts["ELY_ORDER_TORCH"]) == _lib.ORDER_TORCH
    assert int(consts["ELY_EINVAL"]) == _lib.EINVAL and int(consts["ELY_EWORKSPACE"]) == _lib.EWORKSPACE
    assert ctypes.sizeof(_lib.ElyTensor) == 24 and ctypes.sizeof(_lib.ElyConsts) == 32
    assert ctypes.sizeof(_lib.ElyNormResult) == 16


def test_abi_version(lib):
    assert lib.ely_abi_version() == 1


def test_argument_errors_are_status_codes(lib):
    from elysium_wan_amd import _lib

    st = lib.ely_fp8_quantize(None, _lib.BF16, 4, 8, 7, None, None, None, 0, None)
    assert st == _lib.EINVAL and b"fp8 format" in lib.ely_last_error()
    st = lib.ely_fp8_dequantize(None, None, 4, 8, _lib.E4M3, None, 9, None)
    assert st == _lib.EINVAL and b"out_dtype" in lib.ely_last_error()
    st = lib.ely_fp8_quantize(None, _lib.BF16, -1, 8, _lib.E4M3, None, None, None, 0, None)
    assert st == _lib.EINVAL
    st = lib.ely_adamw_step(None, None, None, None, None, -1, None, 0, 0, None, None, 0, None)
    assert st == _lib.EINVAL and b"negative tensor count" in lib.ely_last_error()
    arr = _lib.tensor_array([_lib.ElyTensor(None, 5, _lib.F32, 0)])
    st = lib.ely_grad_norm(arr, 1, 1.0, None, None, 0, None)
    assert st == _lib.EINVAL and b"null pointer" in lib.ely_last_error()
    assert lib.ely_set_max_blocks(-1) == _lib.EINVAL
    assert lib.ely_cast_bf16(None, None, -3, None) == _lib.EINVAL
    assert lib.ely_fold_add(None, None, 5, 4, None) == _lib.EINVAL
    assert lib.ely_selftest_fp8_cvt(0, 1 << 33, 0, None, None) == _lib.EINVAL
    assert lib.ely_selftest_fp8_scaled(0, None, None) == _lib.EINVAL
    assert lib.ely_selftest_fp8_scaled(7, None, None) == _lib.EINVAL
    assert lib.ely_host_device_pointer(None, ctypes.byref(ctypes.c_void_p())) == _lib.EINVAL


def test_argument_errors_of_the_fold_wire_and_recover_entry_points(lib):
    """Every check fails before the HIP runtime is touched."""
    from elysium_wan_amd import _lib

    one = _lib.tensor_array([_lib.ElyTensor(1 << 20, 5, _lib.F32, 0)])
    bf = _lib.tensor_array([_lib.ElyTensor(1 << 20, 5, _lib.BF16, 0)])
    c = (_lib.ElyConsts * 1)()
    st = lib.ely_adamw_fold_step(one, None, bf, one, one, None, 1, c, 0, 0, None, None, 0, None)
    assert st == _lib.EINVAL and b"accumulator" in lib.ely_last_error()
    st = lib.ely_adamw_fold_step(one, bf, bf, one, one, None, 1, c, 0, 0, None, None, 0, None)
    assert st == _lib.EINVAL and b"must be fp32" in lib.ely_last_error()
    short = _lib.tensor_array([_lib.ElyTensor(1 << 20, 4, _lib.F32, 0)])
    st = lib.ely_grad_norm_fold(short, bf, 1, 1.0, None, None, 0, None)
    assert st == _lib.EINVAL and b"numel" in lib.ely_last_error()
    assert lib.ely_grad_norm_fold(None, bf, 1, 1.0, None, None, 0, None) == _lib.EINVAL
    assert lib.ely_byteplanes_split(None, 10, 3, None, None) == _lib.EINVAL
    assert b"esz" in lib.ely_last_error()
    assert lib.ely_byteplanes_split(None, -1, 4, None, None) == _lib.EINVAL
    assert lib.ely_byteplanes_split(None, 10, 4, None, None) == _lib.EINVAL
    assert lib.ely_byteplanes_join(None, 10, 2, None, None) == _lib.EINVAL
    assert lib.ely_byteplanes_split(None, 0, 4, None, None) == _lib.OK  # nothing to do
    assert lib.ely_fp8_nibbles_encode(None, 7, 4, None, None, None, None) == _lib.EINVAL
    assert lib.ely_fp8_nibbles_encode(None, _lib.F32, 4, None, None, None, None) == _lib.EINVAL
    assert lib.ely_fp8_nibbles_decode(None, None, 4, None, None) == _lib.EINVAL
    assert lib.ely_fp8_recover_exp(None, _lib.BF16, 2, 8, 9, None, None, None, 0, None) == _lib.EINVAL
    assert lib.ely_fp8_recover_exp(None, _lib.BF16, 2, 8, _lib.E4M3, None, None, None, 0, None) == _lib.EINVAL
    assert lib.ely_fp8_quantize_k(None, _lib.F32, 2, 8, _lib.E5M2, None, None, None) == _lib.EINVAL
    fake = 1 << 20  # never dereferenced: every call below fails its checks first
    assert lib.ely_fp8_recover_image(None, _lib.BF16, 2, 8, 9, None, None, None, None, 0, None) == _lib.EINVAL
    assert lib.ely_fp8_recover_image(None, 3, 2, 8, _lib.E4M3, None, None, None, None, 0, None) == _lib.EINVAL
    assert lib.ely_fp8_recover_image(fake, _lib.BF16, 2, 8, _lib.E4M3, fake, None, fake, fake, 1 << 20, None) == _lib.EINVAL
    assert b"null pointer" in lib.ely_last_error()
    assert lib.ely_fp8_recover_image(fake, _lib.BF16, 2, 8, _lib.E4M3, fake, fake, fake, fake, 1, None) == _lib.EWORKSPACE
    assert lib.ely_fp8_recover_image(None, _lib.BF16, 0, 8, _lib.E4M3, None, None, None, None, 0, None) == _lib.OK


def test_workspace_queries_are_host_arithmetic(lib):
    from elysium_wan_amd import _lib

    arr = _lib.tensor_array([_lib.ElyTensor(None, 16384 * 3 + 1, _lib.BF16, 0), _lib.ElyTensor(None, 7, _lib.F32, 0)])
    need = lib.ely_grad_norm_workspace_bytes(arr, 2)
    assert need >= 5 * 8 and need % 256 == 0
    assert lib.ely_grad_norm_workspace_bytes(arr, -1) == -1
    # the one-call clip refuses what the norm refuses
    res = ctypes.c_void_p(1)
    assert lib.ely_grad_norm_clip(None, 2, 1.0, res, None, 0, None) == _lib.EINVAL
    fake = _lib.tensor_array([_lib.ElyTensor(16, 16384 * 3 + 1, _lib.BF16, 0), _lib.ElyTensor(16, 7, _lib.F32, 0)])
    assert lib.ely_grad_norm_clip(fake, 2, 1.0, res, res, need - 1, None) == _lib.EWORKSPACE  # refused before any access
    assert lib.ely_adamw_workspace_bytes(192) >= 192 * (64 + 32)
    assert lib.ely_fp8_workspace_bytes(16384, 2560, _lib.BF16) >= 16384 * 4
    # row maxima plus at most 2,048 partial maxima, whatever the row length
    assert lib.ely_fp8_workspace_bytes(2, 1 << 40, _lib.BF16) >= 2048 * 4
    assert lib.ely_fp8_workspace_bytes(2, 1 << 40, _lib.BF16) == lib.ely_fp8_workspace_bytes(2, 64, _lib.BF16)
    # a per-tensor row of at least 64 MiB also has room for the sampled-guess
    # path (the hint path's workspace and two words); below that, the split path's
    for dt, n in ((_lib.BF16, 1 << 25), (_lib.F32, 1 << 24)):
        assert lib.ely_fp8_workspace_bytes(1, n, dt) >= lib.ely_fp8_hint_workspace_bytes(n) + 8
        assert lib.ely_fp8_workspace_bytes(1, n - 8, dt) == lib.ely_fp8_workspace_bytes(1, 64, dt)
    assert lib.ely_fp8_workspace_bytes(1, -1, _lib.BF16) == -1
    assert lib.ely_fp8_recover_workspace_bytes(100) >= lib.ely_fp8_workspace_bytes(100, 0, _lib.BF16) + 400


def test_python_surface_fails_loudly_off_the_gpu():
    from elysium_wan_amd import fp8, optim, pieces

    x = torch.randn(4, 32)
    with pytest.raises(ValueError, match="GPU"):
        fp8.quantize(x)
    with pytest.raises(ValueError, match="GPU"):
        fp8.roundtrip(x.bfloat16(), "e5m2")
    with pytest.raises(ValueError, match="GPU"):
        optim.build("adamw-host", [torch.zeros(3, requires_grad=True)], 1e-3)
    with pytest.raises(ValueError, match="fp32"):
        optim.build("adamw-host", [torch.zeros(3, dtype=torch.bfloat16, requires_grad=True)], 1e-3)
    with pytest.raises(ValueError, match="not one of"):
        optim.build("sgd", [], 1e-3)
    with pytest.raises(ValueError, match="GPU"):
        pieces.cast_piece(x, torch.bfloat16)
    with pytest.raises(ValueError, match="not one of"):
        fp8.quantize(x, "e3m4")


def test_optimizer_bookkeeping_matches_the_reference():
    from elysium_wan_amd import optim

    assert optim.OPTIMIZERS == ("adamw", "adamw-host")
    assert optim.state_bytes_per_param("adamw-host") == 8 and optim.state_bytes_per_param() == 16
    assert optim.hparams(1e-3, "adamw-host")["moments"] == "host"
    assert "moments" not in optim.hparams(1e-3)
    assert optim.ADAMW == {"betas": (0.9, 0.95), "eps": 1e-8, "weight_decay": 0.0}


def test_recipes_refuse_what_the_reference_refuses():
    """"adamw" is torch.optim.AdamW in the reference (runtime/optim.py:50-51):
    the same ValueError, message for message, as torch's own AdamW on the
    same arguments, including an empty parameter list (the ZeRO-1 owner of
    no tensor, integration/test_zero1_empty_shard.py).  "adamw-host" checks
    neither, as HostAdamW: over [] it builds, steps nothing and round-trips
    an empty state."""
    from elysium_wan_amd import optim

    p = [torch.zeros(1, requires_grad=True)]
    for params, kw in ((p, {"lr": -1.0}), (p, {"lr": float("nan")}), (p, {"lr": 1e-3, "eps": -1.0}),
                       (p, {"lr": 1e-3, "betas": (1.0, 0.9)}), (p, {"lr": 1e-3, "betas": (0.9, -0.1)}),
                       (p, {"lr": 1e-3, "weight_decay": -0.1}), ([], {"lr": 1e-3}), ([], {"lr": -1.0})):
        with pytest.raises(ValueError) as want:
            torch.optim.AdamW(params, **{**optim.ADAMW, **kw})
        with pytest.raises(ValueError) as got:
            optim.build("adamw", params, **kw)
        assert str(got.value) == str(want.value)
    host = optim.build("adamw-host", [], 1e-3)
    # the reference's runtime gates promote() on isinstance(opt, optim.HostAdamW) (runtime/stage.py:3134)
    assert isinstance(host, optim.HostAdamW) and host.moments == "host" and host.order == "host"
    assert not isinstance(optim.build("adamw", [torch.zeros(1)], 1e-3), optim.HostAdamW)  # a frozen tensor: no GPU needed
    assert optim.HostAdamW([], 1e-3, moments="device").moments == "device"
    host.step()
    sd = host.state_dict()
    assert sd["state"] == {} and sd["param_groups"][0]["params"] == [] and sd["param_groups"][0]["moments"] == "host"
    host.load_state_dict(sd)


def test_host_constants_equal_the_reference_golden():
    """The package's own constant code (not the oracle's) against the
    constants HostAdamW.step computed in the reference."""
    from conftest import golden
    from elysium_wan_amd import optim

    g = golden("host_adamw.npz")
    for case in ("unit", "decay", "c0"):
        lr, b1, b2, eps, wd, steps = g[f"{case}_hyper"]
        for step in range(int(steps)):
            c = optim.host_consts(lr, (b1, b2), eps, wd, float(step + 1))
            assert [float(x) for x in g[f"{case}_consts"][step][0]] == c


def test_a_missing_library_fails_loudly():
    """No fallback: without libelyhip.so the package raises instead of
    computing anything another way."""
    import subprocess
    import sys

    code = (
        "import sys; sys.path.insert(0, %r)\n"
        "from elysium_wan_amd import _lib\n"
        "try:\n"
        "    _lib.load('/nonexistent/libelyhip.so')\n"
        "except RuntimeError as e:\n"
        "    print('raised', 'build the HIP library' in str(e))\n"
    ) % ROOT
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.stdout.strip() == "raised True", r.stdout + r.stderr


C_CALLER = r"""
#include <stdio.h>
#include <string.h>
#include "ely.h"

int main(void) {
    ely_tensor g[2];
    memset(g, 0, sizeof g);
    g[0].numel = 16384 * 3 + 1;
    g[0].dtype = ELY_BF16;
    g[1].numel = 7;
    g[1].dtype = ELY_F32;
    int64_t ws = ely_grad_norm_workspace_bytes(g, 2);
    int rc = ely_cast_bf16(NULL, NULL, -1, NULL);
    printf("%d %d %lld %d %s\n", (int)ely_abi_version(), rc, (long long)(ws > 0 && ws % 256 == 0),
           (int)(ely_adamw_workspace_bytes(-1) == -1), ely_last_error());
    return 0;
}
"""


def test_header_is_c_and_links_from_c(tmp_path):
    """include/ely.h is a C header: a C11 program (gcc -std=c11 -pedantic
    -Werror) includes it, links libelyhip.so and calls entry points that
    need no GPU -- the binding a C, cgo or JNI caller would start from."""
    import shutil
    import subprocess

    from elysium_wan_amd import _lib

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("no gcc")
    so = _lib.LIB_PATH
    src = tmp_path / "caller.c"
    src.write_text(C_CALLER)
    exe = tmp_path / "caller"
    cmd = [gcc, "-std=c11", "-Wall", "-Wextra", "-pedantic", "-Werror", "-I", os.path.join(ROOT, "include"), str(src),
           "-o", str(exe), so, f"-Wl,-rpath,{os.path.dirname(so)}"]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    version, rc, ws_ok, neg_ok, msg = r.stdout.split(" ", 4)
    assert (int(version), int(rc), int(ws_ok), int(neg_ok)) == (1, _lib.EINVAL, 1, 1)
    assert "negative n" in msg


def test_adamw_refuses_more_tiles_than_its_descriptors_hold(lib):
    """A call whose tensors add up to more than 2^31 - 1 tiles of 256
    elements (the descriptors keep the first tile of each tensor in 32 bits)
    is refused before anything is launched: the pointers below are never
    dereferenced."""
    from elysium_wan_amd import _lib

    fake = 1 << 20
    n = 256 * (1 << 30)  # 2^30 tiles each: the second tensor crosses the limit
    t = _lib.tensor_array([_lib.ElyTensor(fake, n, _lib.F32, 0)] * 2)
    g = _lib.tensor_array([_lib.ElyTensor(fake, n, _lib.BF16, 0)] * 2)
    c = (_lib.ElyConsts * 2)()
    ws = lib.ely_adamw_workspace_bytes(2)
    st = lib.ely_adamw_step(t, g, t, t, None, 2, c, _lib.ORDER_HOST, 0, None, fake, ws, None)
    assert st == _lib.EINVAL and b"tiles" in lib.ely_last_error()


def test_argument_errors_of_the_row_entry_points(lib):
    """The tied fold's row entry points check their arguments before the
    HIP runtime is touched; the pointers below are never dereferenced."""
    from elysium_wan_amd import _lib

    fake = 1 << 20
    assert lib.ely_rows_fold(fake, fake, None, None, None, fake, 4, 8, 8, 0, 16, 7, 0, None) == _lib.EINVAL
    assert b"dtype" in lib.ely_last_error()
    assert lib.ely_rows_fold(None, fake, None, None, None, fake, 4, 8, 8, 0, 16, _lib.F32, 0, None) == _lib.EINVAL
    assert lib.ely_rows_fold(fake, fake, None, None, fake, fake, 4, 8, 8, 0, 16, _lib.F32, 0, None) == _lib.EINVAL
    assert b"b_rows without b" in lib.ely_last_error()
    assert lib.ely_rows_fold(fake, fake, None, fake, None, fake, 4, 8, 8, 2, 16, _lib.F32, 0, None) == _lib.EINVAL
    assert b"compact b" in lib.ely_last_error()
    assert lib.ely_rows_fold(fake, fake, None, None, None, fake, 4, 8, 2, 0, 16, _lib.F32, 0, None) == _lib.EINVAL
    assert lib.ely_rows_fold(None, None, None, None, None, None, 0, 8, 0, 0, 16, _lib.F32, 0, None) == _lib.OK
    assert lib.ely_rows_split(fake, fake, None, fake, 8, 2, 16, _lib.F32, 1, None) == _lib.EINVAL
    assert lib.ely_rows_split(fake, fake, fake, None, 8, 2, 16, _lib.F32, 1, None) == _lib.EINVAL
    assert b"null pointer" in lib.ely_last_error()
    assert lib.ely_rows_split(fake, fake, fake, fake, 8, 2, 16, 9, 1, None) == _lib.EINVAL
    assert lib.ely_rows_split(fake, fake, fake, fake, 8, 9, 16, _lib.BF16, 1, None) == _lib.EINVAL
    assert b"more held rows" in lib.ely_last_error()
    assert lib.ely_rows_split(fake, fake, fake, fake, -1, 0, 16, _lib.BF16, 1, None) == _lib.EINVAL
    assert lib.ely_rows_split(None, None, None, None, 0, 0, 16, _lib.F32, 1, None) == _lib.OK


def _compress_in_child(q, bufs):
    from elysium_wan_amd import planes

    q.put(planes._compress_all(bufs))


def test_plane_compression_keeps_the_serial_bytes_and_survives_a_fork():
    """The byte planes go through zlib on host threads; the blobs are the
    serial ones, in order, and a forked child (whose copy of the parent's
    pool has no threads) compresses with a pool of its own."""
    import multiprocessing as mp
    import zlib

    import numpy as np

    from elysium_wan_amd import planes

    rng = np.random.default_rng(5)
    bufs = [rng.integers(0, 4, size=(1 << 19) + j, dtype=np.uint8) for j in range(4)]
    serial = [zlib.compress(b, 1) for b in bufs]
    assert planes._compress_all(bufs) == serial  # the parent's pool now exists
    ctx = mp.get_context("fork")
    q = ctx.Queue()
    p = ctx.Process(target=_compress_in_child, args=(q, bufs))
    p.start()
    got = q.get(timeout=60)
    p.join(timeout=60)
    assert p.exitcode == 0
    assert got == serial


def test_argument_errors_of_the_hint_entry_point(lib):
    """ely_fp8_quantize_hint refuses bad arguments and a short workspace with
    status codes before the HIP runtime is touched; its workspace query is
    host arithmetic, never below the split path's (its fallback)."""
    from elysium_wan_amd import _lib

    fake = 1 << 20  # never dereferenced
    q = lib.ely_fp8_quantize_hint
    assert q(fake, _lib.BF16, 64, 9, 0, None, fake, fake, None, None, fake, 1 << 20, None) == _lib.EINVAL
    assert b"fp8 format" in lib.ely_last_error()
    assert q(fake, 7, 64, _lib.E4M3, 0, None, fake, fake, None, None, fake, 1 << 20, None) == _lib.EINVAL
    assert q(fake, _lib.BF16, -8, _lib.E4M3, 0, None, fake, fake, None, None, fake, 1 << 20, None) == _lib.EINVAL
    assert q(fake, _lib.BF16, 64, _lib.E4M3, 0, None, fake, None, None, None, fake, 1 << 20, None) == _lib.EINVAL
    assert b"null k" in lib.ely_last_error()
    assert q(fake, _lib.BF16, 64, _lib.E4M3, 0, None, None, fake, None, None, fake, 1 << 20, None) == _lib.EINVAL
    assert b"neither q nor out" in lib.ely_last_error()
    assert q(fake, _lib.BF16, 1 << 24, _lib.E4M3, 3, None, fake, fake, None, None, fake, 256, None) == _lib.EWORKSPACE
    assert b"ely_fp8_hint_workspace_bytes" in lib.ely_last_error()
    ws = lib.ely_fp8_hint_workspace_bytes
    assert ws(-1) == -1
    assert ws(0) >= lib.ely_fp8_workspace_bytes(1, 0, _lib.BF16)
    assert ws(1 << 29) >= (1 << 29) // 2048 * 4 and ws(1 << 29) >= ws(1 << 20)
