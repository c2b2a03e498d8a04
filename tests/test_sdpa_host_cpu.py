"""CPU checks of the SDPA host API (SDPACudaLaunch / SDPACudaBackwardLaunch, the
reference's sdpa/api.hpp:8-31) through the additive _ops_sdpa module: the attribute
defaults and the validation results that fail before any device work."""
import pytest


@pytest.fixture(scope="module")
def sd():
    from graph_executor_v2.ops import _ops_sdpa as s
    return s


def test_attrs_defaults(sd):
    a = sd.SDPAAttrs()
    assert a.scale == 0.0 and not a.causal and a.dropout_p == 0.0 and a.scale_in_train and a.seed == 0


def test_validation(sd):
    q = [2, 2, 8, 64]
    with pytest.raises(RuntimeError, match="Status=1:.*all outputs null"):          # launcher.cu:342
        sd.backward(16, q, 32, q, 48, q, 64)
    with pytest.raises(RuntimeError, match="Status=103"):
        sd.forward(16, q, 32, [2, 2, 8, 32], 48, q, 64, q)                           # K.D != Q.D
    with pytest.raises(RuntimeError, match="Status=103"):
        sd.forward(16, q, 32, q, 48, [2, 2, 9, 64], 64, q)                           # V.N != K.N
    a = sd.SDPAAttrs()
    a.dropout_p = 1.5
    with pytest.raises(RuntimeError, match="Status=4"):                             # dropout_p outside [0, 1]
        sd.forward(16, q, 32, q, 48, q, 64, q, attrs=a, dtype=sd.DType.BF16)
    with pytest.raises(ValueError, match="4D"):
        sd.forward(16, [2, 8, 64], 32, q, 48, q, 64, q)
