"""Reference behaviours at the edges of the API: index wrapping and bounds of
CrossEntropyLoss targets and Embedding indices, the FlashAttention dropout quirk, and
the SGD optimizer state in checkpoints.  GPU only."""
import numpy as np
import pytest
import torch

import oracle as O
from conftest import RTOL_F16, RTOL_F32, assert_close

pytestmark = pytest.mark.gpu


@pytest.fixture
def tg(cuda):
    import tensor_gpu_v2
    return tensor_gpu_v2


def test_cross_entropy_negative_targets_wrap(tg):
    """probs[arange(N), targets] (_nn.py:1145-1150): NumPy indexing wraps targets in
    [-C, 0) and raises outside [-C, C); device targets wrap the same way."""
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((6, 9)) * 2).astype(np.float32)
    t = np.array([0, -1, 8, -9, 3, -4])
    want_loss, probs = O.cross_entropy_fwd(x.astype(np.float64), t % 9)
    want_grad = O.cross_entropy_bwd(probs, t % 9)
    for targets in (t, torch.as_tensor(t, device="cuda"), tg.Tensor(t, requires_grad=False)):
        xt = tg.Tensor(x)
        loss = tg.CrossEntropyLoss()(xt, targets)
        loss.backward()
        assert abs(loss.item() - want_loss) < RTOL_F32 * abs(want_loss)
        assert_close(xt.grad, want_grad, RTOL_F32, "CE grad with wrapped targets")
    with pytest.raises(IndexError):
        tg.CrossEntropyLoss()(tg.Tensor(x), np.array([0, 1, 2, 3, 4, 9]))
    with pytest.raises(IndexError):
        tg.CrossEntropyLoss()(tg.Tensor(x), np.array([0, 1, 2, 3, 4, -10]))


def test_embedding_index_bounds(tg):
    """Host indices: negative ones wrap, indices outside [-V, V) raise IndexError as the
    reference's weight.data[idx] does.  Device indices are not checked (that would need
    a device-to-host read): an index outside [-V, V) gathers a zero row and its
    gradient row is dropped (a documented deviation)."""
    V, dim = 10, 4
    emb = tg.Embedding(V, dim)
    w = emb.weight.numpy().astype(np.float64)
    ids = np.array([[1, -1], [3, -10]])
    out = emb(ids)
    assert_close(out.data, w[ids % V], RTOL_F32, "gather with negative indices")
    g = np.arange(16, dtype=np.float32).reshape(2, 2, dim)
    out.backward(g)
    assert_close(emb.weight.grad, O.embedding_bwd(ids % V, g.astype(np.float64), V), RTOL_F32,
                 "scatter-add with negative indices")
    with pytest.raises(IndexError):
        emb(np.array([0, V]))
    with pytest.raises(IndexError):
        emb(np.array([-V - 1]))
    emb.weight.zero_grad()
    dev = torch.tensor([2, V + 5], device="cuda")
    out = emb(dev)
    assert torch.equal(out.data[1], torch.zeros(dim, device="cuda"))
    out.backward(np.ones((2, dim), np.float32))
    want = np.zeros((V, dim))
    want[2] = 1.0
    assert_close(emb.weight.grad, want, RTOL_F32, "out-of-range device index dropped")


def test_flash_dropout_backward_ignores_the_mask(tg):
    """The reference's flash_attention backward (_core.py:1799-1867) recomputes P
    without the dropout mask and never multiplies by keep/(1-p): the gradients with
    dropout_p > 0 equal those with dropout_p = 0 (the forward output differs)."""
    rng = np.random.default_rng(5)
    shape = (1, 2, 40, 64)
    qn, kn, vn, don = (rng.standard_normal(shape).astype(np.float16) for _ in range(4))
    grads, outs = [], []
    for p in (0.0, 0.5):
        q, k, v = (tg.Tensor(a) for a in (qn, kn, vn))
        o = tg.flash_attention(q, k, v, dropout_p=p)
        o.backward(don)
        grads.append([t.grad.clone() for t in (q, k, v)])
        outs.append(o.data.clone())
    for a, b in zip(*grads):
        assert torch.equal(a, b)
    assert not torch.equal(outs[0], outs[1])
    assert_close(outs[0], O.flash_attention_fwd(*(a.astype(np.float64) for a in (qn, kn, vn)))[0],
                 RTOL_F16, "O without dropout")


def test_sgd_state_in_checkpoint(tg, tmp_path):
    """SGD's momentum velocities are saved and restored with the reference's keys
    (_nn.py:1356-1374)."""
    lin = tg.Linear(5, 3)
    opt = tg.SGD(lin.parameters(), lr=0.1, momentum=0.9, nesterov=True)
    x = tg.Tensor(np.ones((2, 5), np.float32), requires_grad=False)
    lin(x).sum().backward()
    opt.step()
    st = opt.state_dict()
    assert set(st) == {"lr", "momentum", "weight_decay", "nesterov", "velocities"}
    path = str(tmp_path / "sgd.ckpt")
    tg.save_checkpoint(path, lin, optimizer=opt)
    opt2 = tg.SGD(lin.parameters(), lr=0.5)
    tg.load_checkpoint(path, lin, optimizer=opt2)
    assert opt2.lr == 0.1 and opt2.momentum == 0.9 and opt2.nesterov is True
    for a, b in zip(opt.velocities, opt2.velocities):
        assert torch.equal(a, b)
