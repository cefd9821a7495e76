"""attention_softmax_sink (gpu.cuh:201, DeepSeek V4's softmax with a sink) on gfx950, against the oracle — itself
the reference family's door to the bit (tests/test_oracle_ref.py)."""
import numpy as np
import pytest

from silvann_amd import doors
from tests.gpu_util import t
from tests.test_gpu_doors import close

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,length,sink_at", [(64, 2048, 0.0), (5, 33, 9.0), (70000, 3, -3.0)])
def test_softmax_sink(dev, oracle, rows, length, sink_at):
    """attention_softmax_sink (gpu.cuh:201) against the oracle (the reference family's door to the bit); more rows than
    one grid dimension holds."""
    print(f"case: softmax_sink rows{rows} length{length}", flush=True)
    rng = np.random.default_rng(rows + length)
    p = (rng.standard_normal(rows * length) * 3).astype(np.float32)
    sink = (sink_at + rng.standard_normal(rows)).astype(np.float16).view(np.uint16)
    pd = t(p, dev)
    doors.attention_softmax_sink(pd, t(sink, dev), rows, length)
    close(pd.cpu().numpy(), oracle.softmax_sink(p, sink, rows, length), 1e-5)
    assert not doors.launch_failed()
