"""Device output decode (the Parser, parse_model_outputs.py:95-120) against
the oracle's Parser restatement on the same raw output vector."""
import numpy as np
import pytest

from chestnut import Engine
from chestnut import spec as S
from oracle import parse as PR

pytestmark = pytest.mark.gpu

EXTENDED = [['plan', 990], ['lead', 102], ['lead_prob', 3], ['lane_lines', 528], ['lane_lines_prob', 8],
            ['road_edges', 264], ['desire_pred', 32], ['meta', 5], ['pose', 12], ['desire_state', 8],
            ['wide_from_device_euler', 6], ['road_transform', 12], ['extra', 7]]


@pytest.mark.parametrize('outputs', [None, EXTENDED], ids=['default', 'extended'])
def test_decode_matches_parser(gpu, outputs):
    sp = S.get_spec('tiny')
    if outputs:
        sp['outputs'] = outputs
    w = S.make_weights(sp)
    # scale the head weights so logits span a few units (sigmoid/softmax/exp all exercised)
    w['head.w'] = (w['head.w'].astype(np.float32) * 40).astype(np.float16)
    rng = np.random.default_rng(5)
    with Engine(sp, weights=w) as eng:
        packed = eng.PACKED.copy()
        packed[8:10] = (1.0, 0.0)
        for f in range(2):
            warped = rng.integers(0, 256, (2, 6, sp['img_h'], sp['img_w']), dtype=np.uint8)
            out = eng.run_frame(warped, packed)
            got = eng.parsed_outputs()
            ref = PR.parse_outputs({k: out[sl][None] for k, sl in eng.out_slices.items()})
            assert sorted(got) == sorted(ref), (sorted(got), sorted(ref))
            for k in ref:
                assert got[k].shape == ref[k].shape, k
                scale = max(float(np.abs(ref[k]).max()), 1e-30)
                err = float(np.abs(got[k].astype(np.float64) - ref[k]).max()) / scale
                assert err <= 1e-5, (f, k, err)
            packed[12:] = out[eng.out_slices['hidden_state']]
        raw_lead = out[eng.out_slices['lead']]
        print(f"[decode] {'mhp' if raw_lead.size != 144 else 'mdn'} lead, {len(ref)} keys", flush=True)
