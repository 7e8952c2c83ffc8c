"""chestnut.parse: reshaping the device-decoded vector into the Parser's
dictionary (host logic only)."""
import numpy as np

from chestnut.parse import assemble


def test_assemble_shapes_and_keys():
    layout = {
        'plan': {'kind': 'mdn', 'n': 495, 'mu': [0, 495], 'std': [495, 990]},
        'lead_prob': {'kind': 'sigmoid', 'p': [990, 993]},
        'desire_pred': {'kind': 'softmax', 'width': 8, 'p': [993, 1025]},
        'lead': {'kind': 'mhp', 'in_N': 2, 'out_N': 3, 'n': 24, 'weights': [1025, 1031], 'hyp_mu': [1031, 1079],
                 'hyp_std': [1079, 1127], 'mu': [1127, 1199], 'std': [1199, 1271]},
        'odd': {'kind': 'mdn', 'n': 5, 'mu': [1271, 1276], 'std': [1276, 1281]},
        'hidden_state': {'kind': 'raw', 'p': [1281, 1793]},
    }
    dec = np.arange(1793, dtype=np.float32)
    p = assemble(dec, layout)
    assert p['plan'].shape == (1, 33, 15) and p['plan_stds'][0, 0, 0] == 495
    assert p['lead_prob'].shape == (1, 3) and p['desire_pred'].shape == (1, 4, 8)
    assert p['lead_weights'].shape == (1, 2, 3) and p['lead_hypotheses'].shape == (1, 2, 6, 4)
    assert p['lead'].shape == (1, 3, 6, 4) and p['lead_stds'][0, 0, 0, 0] == 1199
    assert p['odd'].shape == (1, 5)                       # unknown head: flat
    np.testing.assert_array_equal(p['hidden_state'][0], dec[1281:])
