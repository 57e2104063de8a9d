"""Front-end contract on the CPU: argument errors, admission, and shape
propagation under FakeTensorMode (no kernel runs).

Follows the reference's contract tests (tests/attention/triangle/
test_triangle_attention.py:455-560, tests/attention/pair_bias/
test_pair_bias_attention.py:488-640): ``ValueError`` for malformed shapes and
mixed dense/nested operands, ``OOpsUnsupportedError`` for CPU tensors,
unsupported dtypes, non-bool masks and forward-mode AD; fake tensors with
(unbacked) symbolic sizes trace through the custom ops.
"""

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode, is_fake
from torch.autograd import forward_ad
from torch.fx.experimental.symbolic_shapes import ShapeEnv

from oops_amd import OOpsUnsupportedError, pair_bias_attention, triangle_attention


class _NestedStandIn:
    """Duck-typed NestedTensor marker (the front-ends detect ``.concat`` + ``.packed_like``)."""

    concat = torch.zeros(1)

    def packed_like(self, values):
        return values


def test_triangle_cpu_tensors_unsupported():
    q = torch.randn(1, 3, 5, 2, 8)
    with pytest.raises(OOpsUnsupportedError):
        triangle_attention(q, q, q)


def test_triangle_shape_errors():
    q = torch.randn(1, 3, 5, 2, 8)
    with pytest.raises(ValueError):
        triangle_attention(q, q, q[..., :-1])
    with pytest.raises(ValueError):
        triangle_attention(q[0, 0], q[0, 0], q[0, 0])  # rank 3
    with pytest.raises(ValueError):
        triangle_attention(q, q, q, torch.ones(1, 4, 5, dtype=torch.bool))
    with pytest.raises(ValueError):
        triangle_attention(q, q, q, None, torch.randn(1, 2, 2, 5, 5))  # bias rows neither 1 nor R


def test_triangle_mixed_nested_is_value_error():
    q = torch.randn(1, 3, 3, 2, 8)
    with pytest.raises(ValueError):
        triangle_attention(q, _NestedStandIn(), q)
    with pytest.raises(ValueError):
        triangle_attention(q, q, q, _NestedStandIn())


def test_triangle_forward_ad_unsupported():
    q = torch.randn(1, 3, 3, 2, 8)
    with forward_ad.dual_level():
        dual = forward_ad.make_dual(q, torch.ones_like(q))
        with pytest.raises(OOpsUnsupportedError):
            triangle_attention(dual, q, q)


def test_pair_bias_contract_on_cpu():
    q = torch.randn(2, 2, 5, 8)
    with pytest.raises(OOpsUnsupportedError):
        pair_bias_attention(q, q, q)
    with pytest.raises(ValueError):
        pair_bias_attention(q, q, q[..., :-1])
    with pytest.raises(ValueError):
        pair_bias_attention(q[0, 0], q[0, 0], q[0, 0])  # rank 2
    with pytest.raises(ValueError):
        pair_bias_attention(q, _NestedStandIn(), q)
    with pytest.raises(OOpsUnsupportedError):  # mask head axis of size 2
        pair_bias_attention(q, q, q, torch.ones(2, 2, 5, 5, dtype=torch.bool))
    with forward_ad.dual_level():
        dual = forward_ad.make_dual(q, torch.ones_like(q))
        with pytest.raises(OOpsUnsupportedError):
            pair_bias_attention(dual, q, q)
    # prefixed (rank 6) shape errors are ValueError, as in the reference
    q6 = torch.randn(2, 2, 3, 2, 5, 8)
    with pytest.raises(ValueError):
        pair_bias_attention(q6, q6, q6, torch.ones(2, 2, 4, 5, dtype=torch.bool))
    with pytest.raises(ValueError):
        pair_bias_attention(q6, q6, q6, None, torch.randn(2, 2, 3, 2, 5, 4))


@pytest.mark.parametrize("layout", ["starting", "ending", "batchless", "prefixed"])
def test_triangle_fake_shapes(layout):
    with FakeTensorMode():
        if layout == "ending":
            q = torch.empty(1, 12, 10, 2, 16, device="cuda", dtype=torch.bfloat16).transpose(1, 2)
        elif layout == "batchless":
            q = torch.empty(10, 12, 2, 16, device="cuda", dtype=torch.bfloat16)
        elif layout == "prefixed":
            q = torch.empty(2, 3, 10, 12, 2, 16, device="cuda", dtype=torch.bfloat16)
        else:
            q = torch.empty(1, 10, 12, 2, 16, device="cuda", dtype=torch.bfloat16)
        rows, cols = q.shape[-4], q.shape[-3]
        bias = torch.empty(*q.shape[:-4], 1, 2, cols, cols, device="cuda", dtype=torch.bfloat16)
        mask = torch.empty(*q.shape[:-4], rows, cols, device="cuda", dtype=torch.bool)
        out = triangle_attention(q, q, q, mask, bias)
        assert is_fake(out)
        assert out.shape == q.shape and out.dtype == q.dtype


def test_pair_bias_fake_unbacked_lengths():
    """The reference's "fake" scenario (test_pair_bias_attention.py:490-506)."""

    shape_env = ShapeEnv()
    query_length = shape_env.create_unbacked_symint()
    key_length = shape_env.create_unbacked_symint()
    torch._check(query_length >= 2)
    torch._check(key_length >= 2)
    with FakeTensorMode(shape_env=shape_env):
        q = torch.empty(2, 2, query_length, 24, device="cuda")
        k = torch.empty(2, 2, key_length, 24, device="cuda")
        mask = torch.empty(2, query_length, key_length, device="cuda", dtype=torch.bool)
        bias = torch.empty(2, 2, query_length, key_length, device="cuda")
        out = pair_bias_attention(q, k, k, mask, bias)
    assert is_fake(out) and out.shape == q.shape and out.dtype == q.dtype


def _nested_qkv(lengths=(3, 5), prefix=()):
    from nested_standin import NestedTensor

    pr = len(prefix)
    tmpl = NestedTensor([torch.empty(*prefix, n, n, 2, 8) for n in lengths], ragged_dims=(pr, pr + 1))
    return [tmpl.packed_like(torch.randn(tmpl.concat.shape)) for _ in range(3)]


def test_nested_contract_on_cpu():
    from nested_standin import NestedTensor

    q, k, v = _nested_qkv()
    with pytest.raises(OOpsUnsupportedError):  # CPU values
        triangle_attention(q, k, v)
    mtmpl = NestedTensor([torch.empty(n, n, dtype=torch.bool) for n in (3, 5)], ragged_dims=(0, 1))
    mask = mtmpl.packed_like(torch.ones(mtmpl.concat.shape, dtype=torch.bool))
    with pytest.raises(ValueError):  # mask orientation differs from q/k/v
        triangle_attention(q, k, v, mask.transpose(-2, -1))
    with pytest.raises(ValueError):  # q/k/v orientations differ
        triangle_attention(q, k.transpose(-4, -3), v)
    k2, _, _ = _nested_qkv(lengths=(4, 4))
    with pytest.raises(ValueError):  # per-sample layouts differ
        triangle_attention(q, k2, v)
    with pytest.raises(ValueError):  # dense mask with nested q/k/v
        triangle_attention(q, k, v, torch.ones(3, 3, dtype=torch.bool))
    with pytest.raises(OOpsUnsupportedError):  # ragged dims that are not the pair axes
        sizes = [(n, 1, 2, n, 8) for n in (3, 5)]
        odd = NestedTensor(ragged_dims=(0, 3), _sizes=sizes, _concat=torch.randn(34, 1, 2, 8))
        triangle_attention(odd, odd, odd)


@pytest.mark.parametrize(
    "make_dout, remapped",
    [
        (lambda s: torch.randn(s), True),  # contiguous (S, H, N, c): the usual upstream gradient
        (lambda s: torch.randn(s[0], s[2], s[1], s[3]).permute(0, 2, 1, 3), True),  # the output's own layout
        (lambda s: torch.randn(s[0], s[1], s[3], s[2]).transpose(-1, -2), False),  # head dim not unit-stride
        (lambda s: torch.randn(1, 1, 1, 1).expand(s), False),  # expanded: copied
    ],
)
def test_dout_table_remap(make_dout, remapped):
    """The backward reads dO through its own table columns when its layout differs from the output's."""

    from oops_amd import _lib
    from oops_amd.attention import _core

    s_, h, n, c = 5, 3, 7, 8
    q = torch.randn(s_, n, h, c).permute(0, 2, 1, 3)  # head-major view of (S, N, H, c) memory
    out = torch.empty_strided(q.size(), q.stride())
    cols = (0, q.stride(0), q.stride(1), q.stride(2))
    table = _core.table_row(groups=s_, len_q=n, len_k=n, q=cols, k=cols, v=cols)
    dout = make_dout(q.shape)
    new = _core._remap_dout(table, out, dout, h)
    assert (new is not None) == remapped
    if new is None:
        return
    off, sg, sh, si = new[_lib.T_DO_OFF : _lib.T_DO_OFF + 4]
    g, hh, i, d = torch.meshgrid(*(torch.arange(x) for x in q.shape), indexing="ij")
    flat = torch.as_strided(dout, (dout.untyped_storage().nbytes() // 4,), (1,), 0)
    got = flat[dout.storage_offset() + off + g * sg + hh * sh + i * si + d]
    torch.testing.assert_close(got, dout, rtol=0, atol=0)
    assert new[: _lib.T_DO_OFF] == table[: _lib.T_DO_OFF]


def test_table_cache_pins_entries_used_under_capture():
    """A geometry table first used while a graph is being captured stays cached (a replay reads its
    device copy) however many other tables follow; ordinary entries are evicted least-recently-used."""

    from oops_amd.attention._core import _TableCache

    made = []
    cache = _TableCache(4, lambda key: made.append(key) or ("host", key, set()))
    captured = cache.get((0, (1, 2)), capturing=True)
    for i in range(600):
        cache.get((0, (i, 9)), capturing=False)
    assert cache.get((0, (1, 2)), capturing=False) is captured
    assert made.count((0, (1, 2))) == 1
    assert len(cache.lru) == 4
    # an entry cached before capture is pinned when a capture uses it
    early = cache.get((0, (7, 7)), capturing=False)
    cache.get((0, (7, 7)), capturing=True)
    for i in range(600, 700):
        cache.get((0, (i, 9)), capturing=False)
    assert cache.get((0, (7, 7)), capturing=False) is early


def test_layer_norm_fake_shapes():
    """Fake tensors outside torch.compile take the custom op's fake kernel (eager calls of real tensors
    go through an autograd.Function instead)."""

    from oops_amd import layer_norm

    with FakeTensorMode():
        x = torch.empty(6, 10, 128, device="cuda", dtype=torch.bfloat16)
        w = torch.empty(128, device="cuda")
        y = layer_norm(x, 128, w, w)
        assert is_fake(y)
        assert y.shape == x.shape and y.dtype == x.dtype


def test_without_second_derivative():
    """Kernel gradients carry a node that raises when differentiated under create_graph=True, and are
    returned unchanged (no node) by an ordinary backward."""

    from oops_amd.attention._runtime import without_second_derivative

    class Square(torch.autograd.Function):
        @staticmethod
        def forward(ctx, x, y):
            ctx.save_for_backward(x)
            return x * x

        @staticmethod
        def backward(ctx, g):
            (x,) = ctx.saved_tensors
            with torch.no_grad():
                gx = 2 * x * g
            return without_second_derivative((gx, None), ctx, g)

    x = torch.randn(5, requires_grad=True)
    (plain,) = torch.autograd.grad(Square.apply(x, None).sum(), x)
    assert plain.grad_fn is None
    (first,) = torch.autograd.grad(Square.apply(x, None).sum(), x, create_graph=True)
    torch.testing.assert_close(first, plain, rtol=0, atol=0)
    with pytest.raises(RuntimeError, match="no second derivatives"):
        first.sum().backward()
