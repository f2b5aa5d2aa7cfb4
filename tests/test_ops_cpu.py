"""torch op surface without a GPU: the reference's schemas are registered
verbatim (patches/glm5-v100-sm70-glue.patch:494-565), fake impls trace, and
CPU tensors are refused (no silent CPU fallback)."""
import pytest
import torch


def test_schemas_registered(pkg, lib):
    ns = pkg.ops.register()
    space = getattr(torch.ops, ns)
    for name, schema in pkg.ops.SCHEMAS.items():
        op = getattr(space, name)
        got = str(op.default._schema)
        want = str(torch._C.parse_schema(f"{ns}::{schema}"))
        assert got == want, (got, want)


def test_fake_impls_trace(pkg, lib):
    from torch._subclasses.fake_tensor import FakeTensorMode

    ns = pkg.ops.register()
    op = getattr(torch.ops, ns).sm70_sparse_mla_decode
    with FakeTensorMode():
        o = torch.empty(2, 64, 512, dtype=torch.float16, device="cuda") if torch.cuda.is_available() \
            else torch.empty(2, 64, 512, dtype=torch.float16)
        # fake mode: no kernel runs, the op only has to accept the schema
        args = [o, torch.empty(2, 64), torch.empty(2, 64, 576, dtype=torch.float16),
                torch.empty(4, 64, 656, dtype=torch.uint8), torch.empty(2, 2048, dtype=torch.int32),
                torch.empty(2, 4, dtype=torch.int32), torch.empty(2, dtype=torch.int32)]
        args = [a.to(o.device) for a in args]
        assert op(*args, 0.04) is None


def test_cpu_tensors_are_refused(pkg, lib):
    ops = pkg._sm70_ops
    y = torch.empty(1, 128, dtype=torch.float16)
    x = torch.empty(1, 128, dtype=torch.float16)
    w = torch.empty(128, 128, dtype=torch.uint8)
    s = torch.empty(1, 1)
    with pytest.raises((NotImplementedError, RuntimeError)):
        ops.sm70_attn_fp8_gemv(y, x, w, s)


def test_missing_op_raises_like_reference(pkg):
    with pytest.raises(RuntimeError, match="not available"):
        pkg._sm70_ops._op("sm70_no_such_op")


def test_cache_writer_in_vllm_namespace(pkg, lib):
    """register_cache_ops puts only the latent-cache writer in the namespace
    vLLM's _custom_ops.concat_and_cache_mla resolves."""
    ns = pkg.ops.register_cache_ops("_mi355_test_cache_ops")
    space = getattr(torch.ops, ns)
    got = str(space.concat_and_cache_mla.default._schema)
    want = str(torch._C.parse_schema(f"{ns}::{pkg.ops.SCHEMAS['concat_and_cache_mla']}"))
    assert got == want
    assert not hasattr(space, "sm70_sparse_mla_decode")
    kv = torch.empty(4, 512, dtype=torch.float16)
    with pytest.raises((NotImplementedError, RuntimeError)):
        space.concat_and_cache_mla(kv, torch.empty(4, 64, dtype=torch.float16),
                                   torch.empty(1, 64, 656, dtype=torch.uint8),
                                   torch.zeros(4, dtype=torch.int64), "fp8_ds_mla",
                                   torch.ones(()))
