"""Write the golden fixtures replayed by the tests (run from the repo root):

    python tests/golden/make_golden.py

Inputs are drawn from fixed seeds; expected outputs come from the NumPy oracle
in float64 (the oracle itself is pinned against torch float64 autograd,
finite differences and known answers in tests/test_oracle.py).  Fixtures are
small .npz files with no pickled objects (np.load(allow_pickle=False)).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle as O  # noqa: E402


def f32(a):
    return np.asarray(a, dtype=np.float32)


def save(name, **arrays):
    # expected values are stored rounded to float32 (6e-8 relative, far inside every
    # tolerance); scalars keep float64
    arrays = {k: (v.astype(np.float32) if isinstance(v, np.ndarray) and v.dtype == np.float64
                  and v.ndim > 0 else v) for k, v in arrays.items()}
    np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrays)


def main():
    rng = np.random.default_rng(20240601)
    # elementwise: a ragged length (not a multiple of the 16-byte vector)
    x = f32(rng.standard_normal(4099) * 2.5)
    dy = f32(rng.standard_normal(4099))
    xd, dyd = x.astype(np.float64), dy.astype(np.float64)
    save("act_bwd", x=x, dy=dy, gelu=O.gelu_bwd(xd, dyd), silu=O.silu_bwd(xd, dyd))

    # softmax over rows of 1000 (not a multiple of 4)
    lg = f32(rng.standard_normal((12, 1000)) * 2)
    y = O.softmax_fwd(lg.astype(np.float64))
    y32 = f32(y)
    dys = f32(rng.standard_normal((12, 1000)))
    save("softmax", logits=lg, y=y, dy=dys,
         dx=O.softmax_bwd(y32.astype(np.float64), dys.astype(np.float64)))

    # layer norm [24, 1024]
    xl = f32(rng.standard_normal((12, 1024)))
    g = f32(1 + 0.02 * rng.standard_normal(1024))
    b = f32(0.02 * rng.standard_normal(1024))
    dyl = f32(rng.standard_normal((12, 1024)))
    yl, xh, mean, var = O.layernorm_fwd(xl.astype(np.float64), g.astype(np.float64),
                                        b.astype(np.float64))
    dx, dg, db = O.layernorm_bwd(xh, var, g.astype(np.float64), dyl.astype(np.float64))
    save("layernorm", x=xl, gamma=g, beta=b, dy=dyl, y=yl, mean=mean[..., 0],
         rstd=1 / np.sqrt(var[..., 0] + 1e-5), dx=dx, dgamma=dg, dbeta=db)

    # FusedBatchNormReLU NHWC [4, 6, 5, 36]
    xb = f32(rng.standard_normal((4, 6, 5, 36)))
    gb = f32(1 + 0.1 * rng.standard_normal(36))
    bb = f32(0.1 * rng.standard_normal(36))
    dyb = f32(rng.standard_normal(xb.shape))
    yb, cache = O.batchnorm_relu_fwd_nhwc(xb.astype(np.float64), gb.astype(np.float64),
                                          bb.astype(np.float64))
    dxb, dgb, dbb = O.batchnorm_relu_bwd_nhwc(dyb.astype(np.float64), gb.astype(np.float64),
                                              cache)
    save("bn_relu_nhwc", x=xb, gamma=gb, beta=bb, dy=dyb, y=yb, dx=dxb, dgamma=dgb, dbeta=dbb)

    # AdamW, three steps
    p = f32(rng.standard_normal(1001))
    m = np.zeros(1001)
    v = np.zeros(1001)
    grads = [f32(rng.standard_normal(1001) * 1e-2) for _ in range(3)]
    pp = p.astype(np.float64)
    for t, gg in enumerate(grads, start=1):
        pp, m, v, _ = O.adam_step(pp, gg.astype(np.float64), m, v, t, lr=3e-4, weight_decay=0.1)
    save("adamw3", p0=p, g=np.stack(grads), p=pp, m=m, v=v)

    # flash attention fp16 inputs, B=1,H=2,S=96,D=64, causal and not
    q = rng.standard_normal((1, 2, 96, 64)).astype(np.float16)
    k = rng.standard_normal((1, 2, 96, 64)).astype(np.float16)
    vv = rng.standard_normal((1, 2, 96, 64)).astype(np.float16)
    do = rng.standard_normal((1, 2, 96, 64)).astype(np.float16)
    out = {"q": q, "k": k, "v": vv, "do": do}
    for causal in (False, True):
        tag = "causal" if causal else "full"
        args = [a.astype(np.float64) for a in (q, k, vv)]
        o, lse = O.flash_attention_fwd(*args, is_causal=causal)
        dq, dk, dv = O.flash_attention_bwd(*args, do.astype(np.float64), is_causal=causal)
        out.update({f"o_{tag}": o, f"lse_{tag}": lse, f"dq_{tag}": dq, f"dk_{tag}": dk,
                    f"dv_{tag}": dv})
    save("flash_attn", **out)

    # C1 MLP: legacy global RNG seed 0, draw order x, w1, w2 (inputs regenerate from the seed)
    np.random.seed(0)
    xm = np.random.randn(32, 784).astype(np.float32)
    w1 = np.random.randn(784, 256).astype(np.float32) * np.float32(np.sqrt(2.0 / 784))
    w2 = np.random.randn(256, 10).astype(np.float32) * np.float32(np.sqrt(2.0 / 256))
    r = O.mlp_step(xm, w1, np.zeros(256, np.float32), w2, np.zeros(10, np.float32))
    sel = np.random.default_rng(1).choice(784 * 256, 2048, replace=False)
    save("mlp_c1", loss=np.array(r["loss"]), dw2=r["dw2"], db1=r["db1"], db2=r["db2"],
         w2=r["w2"], b1=r["b1"], b2=r["b2"], dw1_idx=sel, dw1_sel=r["dw1"].reshape(-1)[sel],
         w1_sel=r["w1"].reshape(-1)[sel], dw1_sum=np.array(r["dw1"].sum()),
         dw1_sq=np.array((r["dw1"] ** 2).sum()))
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
