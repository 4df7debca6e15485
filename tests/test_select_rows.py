"""select_rows (the audited-row selection whose gradient is added into the source tensor's own
accumulated gradient by a hook) against index_select, on the CPU: same values and gradients,
and a loud error when the source receives no other gradient."""
import pytest
import torch

from rte_amd.kernels import hip_ops


def _grads(select, idx, n_sel=1):
    torch.manual_seed(0)
    w = torch.randn(6, 4, 8, dtype=torch.float32, requires_grad=True)
    c = torch.randn(6, 4, 8)
    x = w * 1.5 + 0.25  # non-leaf source, as h0 and the hot hidden state are
    loss = (torch.tanh(x) * c).sum()  # the source's main consumer
    outs = []
    for j in range(n_sel):
        sel = select(x, idx)
        outs.append(sel.detach().clone())
        loss = loss + (sel * sel * (j + 1)).sum()
    loss.backward()
    return w.grad.clone(), outs


@pytest.mark.parametrize("idx", [[2], [0, 5], [3, 3, 1]])
@pytest.mark.parametrize("n_sel", [1, 2])
def test_select_rows_matches_index_select(idx, n_sel):
    ix = torch.tensor(idx, dtype=torch.long)
    g_ref, o_ref = _grads(lambda x, i: x.index_select(0, i), ix, n_sel)
    g_new, o_new = _grads(hip_ops.select_rows, ix, n_sel)
    for a, b in zip(o_ref, o_new):
        assert torch.equal(a, b)
    # one main consumer: every selected row's gradient is the same two-or-more terms in the same
    # order of addition for a single selection; allow rounding when two selections add in
    assert torch.allclose(g_new, g_ref, rtol=1e-6, atol=1e-6)
    if n_sel == 1 and len(set(idx)) == len(idx):
        assert torch.equal(g_new, g_ref)


def test_select_rows_without_other_consumer_raises():
    """The source's only gradient would be the selected rows': no hook may supply it, so the
    backward fails loudly instead of dropping the rows."""
    w = torch.randn(4, 3, requires_grad=True)
    sel = hip_ops.select_rows(w * 2.0, torch.tensor([1]))
    with pytest.raises(RuntimeError, match="select_rows"):
        sel.sum().backward()


def test_select_rows_no_grad_and_leaf_fall_back():
    w = torch.randn(4, 3, requires_grad=True)
    ix = torch.tensor([2, 0])
    assert torch.equal(hip_ops.select_rows(w, ix), w.index_select(0, ix))
    assert hip_ops.select_rows(w, ix).grad_fn.name().startswith("IndexSelect")
    with torch.no_grad():
        assert hip_ops.select_rows(w * 2, ix).grad_fn is None


@pytest.mark.parametrize("a_first", [True, False])
def test_select_rows_pass_through_gradient_not_written(a_first):
    """The source's other consumer is a residual add, whose backward hands the same gradient
    tensor to both of its inputs: adding the selected rows must not write into it, or the other
    input's gradient would carry them too (it does when the sibling's backward runs after the
    hook, i.e. when the source is created last)."""
    def run(select):
        torch.manual_seed(1)
        wa = torch.randn(5, 4, requires_grad=True)
        wb = torch.randn(5, 4, requires_grad=True)
        if a_first:  # non-leaf sources, in both creation orders
            a = wa * 2.0
            b = wb * 3.0
        else:
            b = wb * 3.0
            a = wa * 2.0
        z = a + b                   # AddBackward passes one gradient to a and b
        loss = (z * torch.randn(5, 4)).sum()
        sel = select(a, torch.tensor([1, 3]))
        loss = loss + (sel * sel).sum()
        loss.backward()
        return wa.grad.clone(), wb.grad.clone()

    ga_ref, gb_ref = run(lambda x, i: x.index_select(0, i))
    ga, gb = run(hip_ops.select_rows)
    assert torch.allclose(ga, ga_ref, rtol=1e-6, atol=1e-6)
    assert torch.equal(gb, gb_ref)
