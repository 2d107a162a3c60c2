"""Replay-buffer record handling on the CPU (hive_fnn/fnn_replay_buffer.py
counterpart): the opening-value merge."""
import numpy as np

from hive_neuralnet_amd.orchestrator import FNNTrainingExample
from hive_neuralnet_amd.replay import compact_opening_value_examples


def _ex(turn, tag, value, w=1.0, use_v=True):
    s = np.zeros(3424, np.uint8)
    s[3412] = turn
    s[0] = tag
    return FNNTrainingExample(s, np.array([1.0], np.float32), value, True, use_v, w)


def test_opening_value_merge():
    a1, a2, a3 = _ex(1, 7, 1.0, 1.0), _ex(1, 7, -1.0, 3.0), _ex(1, 7, 1.0, 0.0)
    late = _ex(9, 7, 1.0)
    lone = _ex(2, 5, -1.0)
    novalue = _ex(0, 7, 1.0, use_v=False)
    out = compact_opening_value_examples([a1, late, a2, lone, novalue, a3], 4)
    # ungrouped first, in input order; then the groups in order of first occurrence: a repeated
    # position's members without value, then its merged value example; a lone position as is
    assert out[0] is late and out[1] is novalue and out[6] is lone
    members, merged = out[2:5], out[5]
    assert all(not m.use_for_value and m.use_for_policy for m in members)
    assert merged.use_for_value and not merged.use_for_policy and merged.value_weight == 4.0
    assert abs(merged.value_target - (1.0 * 1 - 1.0 * 3 + 1.0 * 0) / 4.0) < 1e-12
    assert len(out) == 7
    # weights summing to zero average over the count
    z = compact_opening_value_examples([_ex(0, 1, 1.0, 0.0), _ex(0, 1, -0.5, 0.0)], 4)
    assert z[-1].value_weight == 2.0 and z[-1].value_target == 0.0
    assert compact_opening_value_examples([a1, a2], 0) == [a1, a2]
