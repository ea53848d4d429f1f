"""The reference's operator names and schemas are registered (CPU).

The reference's ``torchwarp_udtw`` / ``torchwarp_jeanie`` custom operators
(``udtw/_ops.py:100-211``, ``jeanie/_ops.py:110-230``) must resolve by name,
with the reference's argument names, types and output counts, so code and
exported graphs that call them bind. The expected schemas below are the ones
torch generates from the reference's Python signatures (Python ``int`` is
``SymInt``, ``Optional[Tensor]`` is ``Tensor?``).
"""

import torch

import torchwarp_amd  # noqa: F401  (registers the operators)

EXPECTED = {
    ("torchwarp_udtw", "dp"):
        "torchwarp_udtw::dp(Tensor cost, Tensor penalty, float gamma, float bandwidth, "
        "str backend) -> (Tensor, Tensor, Tensor, Tensor)",
    ("torchwarp_udtw", "dp_backward"):
        "torchwarp_udtw::dp_backward(Tensor cost, Tensor penalty, Tensor R, Tensor P, "
        "Tensor grad_r, Tensor grad_p, float gamma, float bandwidth, str backend) "
        "-> (Tensor, Tensor)",
    ("torchwarp_udtw", "fused"):
        "torchwarp_udtw::fused(Tensor X, Tensor Y, Tensor vx, Tensor vy, float gamma, "
        "float beta, float eps, float bandwidth, str backend) "
        "-> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)",
    ("torchwarp_udtw", "fused_backward"):
        "torchwarp_udtw::fused_backward(Tensor X, Tensor Y, Tensor vx, Tensor vy, Tensor R, "
        "Tensor P, Tensor G, Tensor x2, Tensor y2, Tensor grad_r, Tensor grad_p, float gamma, "
        "float beta, float eps, float bandwidth, str backend) -> (Tensor, Tensor, Tensor, Tensor)",
    ("torchwarp_jeanie", "dp"):
        "torchwarp_jeanie::dp(Tensor cost, SymInt s1, SymInt s2, float gamma, str backend, "
        "bool natural_R) -> (Tensor, Tensor, Tensor)",
    ("torchwarp_jeanie", "dp_backward"):
        "torchwarp_jeanie::dp_backward(Tensor cost, Tensor R_d, Tensor grad_out, "
        "Tensor? grad_R, SymInt s1, SymInt s2, float gamma, str backend) -> Tensor",
    ("torchwarp_jeanie", "features"):
        "torchwarp_jeanie::features(Tensor query, Tensor support, SymInt s1, SymInt s2, "
        "float gamma, SymInt metric, str backend, bool natural_R) "
        "-> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)",
    ("torchwarp_jeanie", "features_backward"):
        "torchwarp_jeanie::features_backward(Tensor query, Tensor support, Tensor R_d, "
        "Tensor G, Tensor q_sq, Tensor s_sq, Tensor grad_out, Tensor? grad_R, SymInt s1, "
        "SymInt s2, float gamma, SymInt metric, str backend) -> (Tensor, Tensor)",
}


def test_reference_operator_schemas():
    for (ns, name), want in EXPECTED.items():
        op = getattr(getattr(torch.ops, ns), name).default
        assert str(op._schema) == want, (ns, name, str(op._schema))


def test_reference_operators_trace_with_fake_tensors():
    """The fake implementations give the outputs' shapes without running a
    kernel (what torch.compile and export use)."""
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        c = torch.empty(3, 5, 7, device="cpu")
        out = torch.ops.torchwarp_udtw.dp(c, c, 1.0, 0.0, "auto")
        assert [tuple(t.shape) for t in out[:2]] == [(3,), (3,)] and out[3].shape == (3, 35)
        g = torch.ops.torchwarp_udtw.dp_backward(c, c, out[2], out[3], out[0], out[1], 1.0, 0.0,
                                                "auto")
        assert g[0].shape == c.shape and g[1].shape == c.shape
        X, Y = torch.empty(3, 5, 4), torch.empty(3, 7, 4)
        vx, vy = torch.empty(3, 5), torch.empty(3, 7)
        f = torch.ops.torchwarp_udtw.fused(X, Y, vx, vy, 1.0, 1.0, 1e-8, 0.0, "auto")
        assert len(f) == 7 and f[4].shape == (3, 35)
        fb = torch.ops.torchwarp_udtw.fused_backward(X, Y, vx, vy, f[2], f[3], f[4], f[5], f[6],
                                                    f[0], f[1], 1.0, 1.0, 1e-8, 0.0, "auto")
        assert [t.shape for t in fb] == [X.shape, Y.shape, vx.shape, vy.shape]
        cj = torch.empty(2, 3, 1, 6, 5)
        o = torch.ops.torchwarp_jeanie.dp(cj, 1, 0, 0.1, "auto", True)
        assert o[0].shape == (2,) and o[2].shape == cj.shape
        assert torch.ops.torchwarp_jeanie.dp_backward(cj, o[1], o[0], None, 1, 0, 0.1,
                                                      "auto").shape == cj.shape
        q, s = torch.empty(2, 3, 1, 6, 8), torch.empty(2, 5, 8)
        fo = torch.ops.torchwarp_jeanie.features(q, s, 1, 0, 0.1, 1, "auto", False)
        assert len(fo) == 6 and fo[3].shape == (2, 3, 1, 6, 5)
        dq, ds = torch.ops.torchwarp_jeanie.features_backward(q, s, fo[1], fo[3], fo[4], fo[5],
                                                              fo[0], None, 1, 0, 0.1, 1, "auto")
        assert dq.shape == q.shape and ds.shape == s.shape
