"""Parsed model outputs: the reference's `Parser.parse_outputs` dictionary
(parse_model_outputs.py:95-120, as modeld.py:161-162 and 195 call it on the
output vector sliced by `output_slices`), assembled from the engine's device
decode.

Every frame plan ends with the decode kernel (decode.hip), which applies the
Parser's per-head treatment on device and leaves the result in the state
tensor "decoded"; `ck_decoded_layout` describes where each head's pieces sit.
This module only reshapes those pieces into the Parser's keys and shapes:

  MDN head NAME   -> NAME (mu), NAME_stds (safe_exp std), shape (1,) + out_shape
  sigmoid head    -> NAME, shape (1, len)
  softmax head    -> NAME, shape (1,) + out_shape
  multi-hypothesis lead -> lead_weights (1, in_N, out_N), lead_hypotheses,
                    lead_stds_hypotheses (1, in_N) + out_shape, lead, lead_stds
                    (1, out_N) + out_shape
  anything else   -> the raw slice, shape (1, len) (modeld.py:162)
"""
import numpy as np

# ModelConstants values the output shapes use (constants.py:8-57)
IDX_N = 33
POSE_WIDTH = 6
WIDE_FROM_DEVICE_WIDTH = 3
LANE_LINES_WIDTH = 2
NUM_LANE_LINES = 4
NUM_ROAD_EDGES = 2
PLAN_WIDTH = 15
DESIRE_PRED_LEN = 4
DESIRE_PRED_WIDTH = 8
LEAD_TRAJ_LEN = 6
LEAD_WIDTH = 4
LEAD_MHP_SELECTION = 3

# per-head out_shape of the Parser's calls (parse_model_outputs.py:96-115)
OUT_SHAPES = {
    'pose': (POSE_WIDTH,),
    'wide_from_device_euler': (WIDE_FROM_DEVICE_WIDTH,),
    'road_transform': (POSE_WIDTH,),
    'lane_lines': (NUM_LANE_LINES, IDX_N, LANE_LINES_WIDTH),
    'road_edges': (NUM_ROAD_EDGES, IDX_N, LANE_LINES_WIDTH),
    'desire_pred': (DESIRE_PRED_LEN, DESIRE_PRED_WIDTH),
    'plan': (IDX_N, PLAN_WIDTH),
    'desire_state': (DESIRE_PRED_WIDTH,),
}
LEAD_SHAPE_MDN = (LEAD_MHP_SELECTION, LEAD_TRAJ_LEN, LEAD_WIDTH)
LEAD_SHAPE_MHP = (LEAD_TRAJ_LEN, LEAD_WIDTH)


def _shape(name, size, mhp=False):
    if name == 'lead':
        s = LEAD_SHAPE_MHP if mhp else LEAD_SHAPE_MDN
    else:
        s = OUT_SHAPES.get(name)
    # a spec may size a head differently from the reference's constants:
    # keep the values flat then
    return s if s is not None and int(np.prod(s)) == size else (size,)


def assemble(decoded, layout):
    """decoded: f32 vector read from the engine; layout: the parsed JSON of
    ck_decoded_layout.  Returns the Parser's output dictionary."""
    out = {}
    for name, L in layout.items():
        k = L['kind']
        if k == 'mdn':
            mu = decoded[L['mu'][0]:L['mu'][1]]
            sd = decoded[L['std'][0]:L['std'][1]]
            s = _shape(name, mu.size)
            out[name] = mu.reshape((1,) + s).copy()
            out[name + '_stds'] = sd.reshape((1,) + s).copy()
        elif k == 'mhp':
            N, S, n = L['in_N'], L['out_N'], L['n']
            s = _shape(name, n, mhp=True)
            out[name + '_weights'] = decoded[L['weights'][0]:L['weights'][1]].reshape(1, N, S).copy()
            out[name + '_hypotheses'] = decoded[L['hyp_mu'][0]:L['hyp_mu'][1]].reshape((1, N) + s).copy()
            out[name + '_stds_hypotheses'] = decoded[L['hyp_std'][0]:L['hyp_std'][1]].reshape((1, N) + s).copy()
            fs = (1, S) + s if S > 1 else (1,) + s
            out[name] = decoded[L['mu'][0]:L['mu'][1]].reshape(fs).copy()
            out[name + '_stds'] = decoded[L['std'][0]:L['std'][1]].reshape(fs).copy()
        elif k == 'softmax':
            p = decoded[L['p'][0]:L['p'][1]]
            out[name] = p.reshape((1,) + _shape(name, p.size)).copy()
        else:   # sigmoid, raw
            out[name] = decoded[L['p'][0]:L['p'][1]].reshape(1, -1).copy()
    return out
