"""SamplerState host logic (parameters, kwargs merge, compaction) on CPU
tensors; sampling itself needs the GPU (tests/test_gpu_state.py)."""

import pytest
import torch

from lps import SamplerState


def test_add_merges_kwargs_and_rejects_unknown_keys():
    st = SamplerState(4, 100, 8, "cpu")
    i = st.add({"temperature": 0.5, "top_k": 7, "presence_penalty": 0.25}, history=[1, 2, 3])
    assert i == 0 and st.n == 1
    assert float(st.params.temperature[0]) == 0.5 and int(st.params.top_k[0]) == 7
    assert float(st.params.presence_penalty[0]) == 0.25
    assert float(st.params.top_p[0]) == pytest.approx(0.9)  # the reference default SamplingConfig.top_p (fp32)
    assert st.history(0) == [1, 2, 3]
    with pytest.raises(TypeError):
        st.add({"no_such_key": 1})
    assert st.n == 1


def test_remove_compacts_in_order():
    st = SamplerState(5, 100, 4, "cpu")
    for t in range(5):
        st.add({"temperature": 0.1 * (t + 1)}, history=[t] * (t % 4 + 1))
    st.remove([1, 3])
    assert st.n == 3
    assert [round(float(x), 3) for x in st.params.temperature[:3]] == [0.1, 0.3, 0.5]
    assert [st.history(i) for i in range(3)] == [[0], [2, 2, 2], [4]]


def test_history_truncated_to_capacity_and_full_state():
    st = SamplerState(1, 100, 3, "cpu")
    st.add(history=list(range(10)))
    assert st.history(0) == [0, 1, 2]
    with pytest.raises(RuntimeError):
        st.add()
