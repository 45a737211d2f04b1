"""The recent window's device moves (one launch to append a block, one to shift
after a flush) against the oracle's window, after every add_recent: blocks of
uneven sizes, Alpha span flags, flush granules smaller than half the window
(the shift then overlaps and takes tensor copies), and sources given as
strided views."""

import numpy as np
import pytest
import torch

from harness import compare_state, make_pair, to_np
from workloads import Mixture

pytestmark = pytest.mark.gpu


def _window_equal(gpu, ora):
    bad = []
    for name in ("recent_k", "recent_k_raw", "recent_v", "recent_pos"):
        if not np.array_equal(to_np(getattr(gpu, name)), np.asarray(getattr(ora, name))):
            bad.append(name)
    if gpu.alpha_exact_tokens:
        ends = np.asarray(ora.recent_ends, dtype=np.uint8)
        if not np.array_equal(to_np(gpu.recent_span_ends).astype(np.uint8), ends):
            bad.append("recent_span_ends")
    if gpu.recent_count != ora.recent_count:
        bad.append("recent_count")
    return bad


@pytest.mark.parametrize("exact,recent,flush,strided", [(0, 64, 64, False), (0, 64, 16, True), (32, 64, 64, True),
                                                        (32, 96, 32, False)])
def test_recent_window_matches_oracle(exact, recent, flush, strided):
    print(f"case exact={exact} recent={recent} flush={flush} strided={strided}", flush=True)
    gpu, ora = make_pair(batch=2, groups=2, dim=64, K=4, B=8, recent=recent, flush=flush, max_seq=1024, s_h=16.0,
                         exact=exact, span=8, beta_novelty=bool(exact), beta_adaptive=bool(exact))
    mix = Mixture(2, 2, 64, clusters=4, seed=13)
    dev = gpu.level_k.device
    start = 0
    for n in (5, 17, 64, 1, 40, 33, 64, 7, 50, 64, 3):
        n = min(n, recent)
        k_raw, v, k = mix.rows(n), mix.rows(n), mix.rows(n)
        pos = torch.arange(start, start + n).unsqueeze(0).expand(2, -1).contiguous()
        ends = mix.span_ends(start, n, 8) if exact else None
        ora.add_recent(k.float().numpy(), v.float().numpy(), k_raw.float().numpy(), pos.numpy(), ends)
        kd, vd, krd = k.to(dev), v.to(dev), k_raw.to(dev)
        if strided:
            # [B, n, G, D] storage seen as [B, G, n, D]: row stride G * D, group stride D.
            kd = kd.transpose(1, 2).contiguous().transpose(1, 2)
            vd = vd.transpose(1, 2).contiguous().transpose(1, 2)
        gpu.add_recent(kd, vd, k_raw=krd, input_pos=pos.to(dev), span_ends=ends)
        torch.cuda.synchronize()
        bad = _window_equal(gpu, ora) + compare_state(gpu, ora)
        assert not bad, f"after {start + n} rows: {bad}"
        start += n
