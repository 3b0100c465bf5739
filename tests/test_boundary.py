"""The drop-in boundary without a GPU.

* Importing ``voyager_amd`` or ``voyager_amd.kernels`` defines nothing, so
  the reference can define ``quantized_ops`` itself afterwards
  (``src/voyager_compiler/ops/quantized.py:97``) and bind this package's
  kernels onto its library with ``kernels.register`` -- including over the
  reference's own torch.compile CUDA kernels (``:100-109``), with
  ``allow_override``.
* ``register`` binds every op's CUDA kernel and fake kernel onto a fresh
  namespace with the same schema strings; the fake kernels propagate shapes
  and dtypes; CPU tensors are refused.

Each scenario that defines ``quantized_ops`` runs in a child interpreter,
since a namespace can be defined once per process.
"""

import os
import subprocess
import sys
import textwrap

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "voyager-compiler-2_amd")


def _child(code: str) -> str:
    env = dict(os.environ, PYTHONPATH=os.pathsep.join([ROOT, PKG, os.environ.get("PYTHONPATH", "")]))
    res = subprocess.run([sys.executable, "-c", textwrap.dedent(code)], capture_output=True, text=True, env=env,
                         timeout=300)
    assert res.returncode == 0, res.stdout + res.stderr
    return res.stdout


def test_import_defines_nothing_and_binds_onto_the_reference_library():
    out = _child("""
        import torch
        import voyager_amd, voyager_amd.kernels as K
        from voyager_amd.schemas import SCHEMAS
        # the reference's module defines the namespace after the import ...
        ref = torch.library.Library("quantized_ops", "DEF")
        for s in SCHEMAS.values():
            ref.define(s)
        # ... and registers its compiled CUDA kernel for a few ops
        ref.impl("quantize", lambda *a, **k: None, "CUDA")
        try:
            K.register(ref)
        except RuntimeError as e:
            print("collision:", "already a kernel registered" in str(e))
        done = K.register(ref, allow_override=True, only=list(SCHEMAS))
        has = [torch._C._dispatch_has_kernel_for_dispatch_key("quantized_ops::" + n, "CUDA") for n in done]
        print("bound", len(done), all(has))
    """)
    assert "collision: True" in out
    assert "bound 17 True" in out


def test_register_onto_a_fresh_namespace():
    out = _child("""
        import torch
        from voyager_amd import kernels, schemas
        lib = torch.library.Library("vh_fresh", "DEF")
        defined = schemas.SCHEMAS | schemas.TWIN_SCHEMAS
        for s in defined.values():
            lib.define(s)
        done = kernels.register(lib, fakes=True)
        # every defined op but the two layout twins, which are torch restatements
        assert sorted(done) == sorted(set(defined) - {"sdpa_kmajor", "rms_norm_kmajor"}), sorted(done)
        ops = torch.ops.vh_fresh
        for n in done:
            assert torch._C._dispatch_has_kernel_for_dispatch_key("vh_fresh::" + n, "CUDA"), n
        # fake kernels: shapes and dtypes through FX-style shape propagation
        m = lambda *s, dt=torch.bfloat16: torch.empty(*s, dtype=dt, device="meta")
        tab = m(65536)
        s, c = ops.quantize_mx(m(8, 100), tab, [-1], 16, 127.0, True)
        assert list(s.shape) == [8, 7] and list(c.shape) == [8, 100]
        s, z, v = ops.quantize_affine(m(2, 64, 128), tab, [-2], 32, 0.0, 3.0)
        assert list(s.shape) == [2, 2, 128] and list(v.shape) == [2, 64, 128]
        y = ops.linear_mx(m(4, 64), m(32, 64), input_scale=m(4, 4), weight_scale=m(32, 4), block_size=16)
        assert list(y.shape) == [4, 32] and y.dtype == torch.bfloat16
        y = ops.linear(m(4, 64), m(32, 64), out_dtype=torch.float32)
        assert list(y.shape) == [4, 32] and y.dtype == torch.float32
        a = ops.sdpa_mx(m(1, 8, 3, 128), m(1, 2, 40, 128), m(1, 2, 40, 128), enable_gqa=True)
        assert list(a.shape) == [1, 8, 3, 128]
        t = ops.quantize_mx_transpose(m(48, 64), tab, 16, 127.0, True)
        assert [list(x.shape) for x in t] == [[48, 4], [48, 64], [64, 3], [64, 48]]
        try:
            ops.quantize_mx(torch.ones(4, 16, dtype=torch.bfloat16), torch.ones(65536), [-1], 16, 127.0, True)
        except (RuntimeError, NotImplementedError) as e:
            print("cpu refused")
        print("ok")
    """)
    assert "cpu refused" in out and "ok" in out


def test_standalone_library_defines_every_schema():
    out = _child("""
        import torch
        import voyager_amd.library
        from voyager_amd import schemas
        for name, s in schemas.all_schemas().items():
            op = getattr(torch.ops.quantized_ops, name).default
            assert str(op._schema) == str(torch._C.parse_schema("quantized_ops::" + s)), name
        # the layout twins run on any device (torch restatements)
        x = torch.randn(2, 8, 5, 6)
        y = torch.ops.quantized_ops.max_pool2d(x.permute(0, 2, 3, 1).contiguous(), [2, 2])
        ref = torch.nn.functional.max_pool2d(x, 2).permute(0, 2, 3, 1)
        assert torch.equal(y, ref)
        h = torch.randn(3, 16, 7)
        w = torch.randn(16, 1)
        got = torch.ops.quantized_ops.rms_norm_kmajor(h, w, 1e-6)
        exp = torch.nn.functional.rms_norm(h.mT, [16], w.reshape(16), 1e-6).mT
        assert torch.allclose(got, exp)
        q, k, v = torch.randn(1, 2, 4, 8), torch.randn(1, 2, 6, 8), torch.randn(1, 2, 6, 8)
        got = torch.ops.quantized_ops.sdpa_kmajor(q.mT, k.mT, v)
        assert torch.allclose(got, torch.nn.functional.scaled_dot_product_attention(q, k, v), atol=1e-6)
        print("ok")
    """)
    assert "ok" in out
