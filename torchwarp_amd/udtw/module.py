"""``nn.Module`` front end for uDTW (drop-in for ``torchwarp.udtw.module``, module.py:8-51)."""

import torch.nn as nn

from .functional import _BACKENDS, _check_hyperparameters, udtw


class UDTW(nn.Module):
    """Module form of ``torchwarp_amd.functional.udtw`` with its settings fixed.

    Constructor settings: ``gamma`` is the soft-minimum temperature (positive);
    ``beta`` weighs the uncertainty penalty (non-negative); ``normalize``
    subtracts half of the two self-alignments, d(X,Y) - [d(X,X) + d(Y,Y)] / 2,
    from both outputs; ``bandwidth`` restricts paths to |i - j| <= bandwidth
    (None or 0: no restriction); ``method`` chooses between building the
    cost inside the HIP kernels ("gemm") and materialising the [B, N, M]
    cost and penalty first ("diff"); ``backend`` is "auto" or "cuda".

    Calling the module on sequences X [B, N, D], Y [B, M, D] and their
    per-step standard deviations sigma_x [B, N, 1], sigma_y [B, M, 1]
    returns ``UDTWOutput(distance, penalty)``, two [B] tensors, the penalty
    already multiplied by beta.
    """

    def __init__(self, gamma=1.0, beta=1.0, normalize=False, bandwidth=None, *,
                 method="gemm", backend="auto"):
        super().__init__()
        self.gamma = float(gamma)
        self.beta = float(beta)
        self.normalize = bool(normalize)
        self.bandwidth = None if bandwidth is None else float(bandwidth)
        if backend not in _BACKENDS:
            raise ValueError("backend must be one of {}".format(_BACKENDS))
        if method not in ("gemm", "diff"):
            raise ValueError("method must be 'gemm' or 'diff'")
        self.method = method
        self.backend = backend
        _check_hyperparameters(self.gamma, self.beta, self.bandwidth)

    def forward(self, X, Y, sigma_x, sigma_y):
        return udtw(X, Y, sigma_x, sigma_y, beta=self.beta, gamma=self.gamma,
                    normalize=self.normalize, bandwidth=self.bandwidth, method=self.method,
                    backend=self.backend)

    def extra_repr(self):
        return "gamma={}, beta={}, normalize={}, bandwidth={}, method={!r}, backend={!r}".format(
            self.gamma, self.beta, self.normalize, self.bandwidth, self.method, self.backend)
