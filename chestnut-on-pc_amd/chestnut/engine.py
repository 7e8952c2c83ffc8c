"""Python surface of the frame engine, mirroring the reference's namespace.

The reference's callers `exec` run_pinned2.py up to '# --- smoke run' and use
`run_frame(warped_np, packed)`, `out_slices`, `img`, `make_warped`, `PACKED`
(run_pinned2.py:1353-1389, 1462-1565; video_check.py:18-19, 59-60).
`Engine` provides the same names over the native library; `load(spec)`
returns a namespace with exactly those attributes.
"""
import ctypes
import json
import types
from collections.abc import Mapping
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from . import spec as _spec
from ._lib import call, lib

_DT = {0: np.float32, 1: np.float16, 2: np.uint8, 3: np.uint32}


class Engine:
    """One model on one GPU: parameters, queues, plan and hipGraph.

    spec: spec name ('driving_39m', 'big_driving_1b', 'tiny') or dict.
    weights: dict name -> array; None generates the seeded weights.
    """

    def __init__(self, spec='big_driving_1b', weights=None, seed=None, graph=True, gen_threads=8):
        self.spec = _spec.get_spec(spec)
        if seed is not None:
            self.spec['seed'] = int(seed)
        h = ctypes.c_void_p()
        call('ck_create', _spec.spec_json(self.spec).encode(), ctypes.byref(h))
        self._h = h
        try:
            self._check_param_table()
            self.upload_weights(weights, gen_threads)
            n = ctypes.c_int()
            call('ck_output_size', self._h, ctypes.byref(n))
            self.n_out = n.value
            buf = ctypes.create_string_buffer(1 << 14)
            call('ck_output_slices', self._h, buf, len(buf))
            self.out_slices = {k: slice(v[0], v[1]) for k, v in json.loads(buf.value.decode()).items()}
            lbuf = ctypes.create_string_buffer(1 << 16)
            call('ck_decoded_layout', self._h, None, lbuf, len(lbuf))
            self.decoded_layout = json.loads(lbuf.value.decode())
            self.set_graph(graph)
        except Exception:
            self.close()
            raise
        s = self.spec
        self.img = (1, 6 * s['n_frames'], s['img_h'], s['img_w'])
        self.PACKED = np.zeros(s['desire_len'] + 4 + s['feat_len'], np.float32)

    # -- lifecycle --------------------------------------------------------------
    def close(self):
        if getattr(self, '_h', None):
            lib().ck_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    # -- parameters -------------------------------------------------------------
    def param_names(self):
        n = ctypes.c_int()
        call('ck_param_count', self._h, ctypes.byref(n))
        out = []
        name = ctypes.create_string_buffer(256)
        nb = ctypes.c_size_t()
        dt = ctypes.c_int()
        for i in range(n.value):
            call('ck_param_info', self._h, i, name, len(name), ctypes.byref(nb), ctypes.byref(dt))
            out.append((name.value.decode(), nb.value, _DT[dt.value]))
        return out

    def _check_param_table(self):
        native = self.param_names()
        table = _spec.param_table(self.spec)
        if [n for n, _, _ in native] != [t[0] for t in table]:
            raise RuntimeError('native and Python parameter tables disagree')
        for (n, nb, dt), (_, shape, tdt, _, _) in zip(native, table):
            want = int(np.prod(shape)) * (2 if tdt == 'f16' else 4)
            if nb != want:
                raise RuntimeError(f'parameter {n}: native {nb} bytes, table {want}')

    def upload_weights(self, weights=None, threads=8):
        """Upload `weights` (or the spec's seeded weights, generated on the fly)."""
        table = _spec.param_table(self.spec)
        seed = self.spec['seed']

        def one(p):
            name = p[0]
            arr = weights[name] if weights is not None else _spec.make_param(seed, *p)
            arr = np.ascontiguousarray(arr, dtype=np.float16 if p[2] == 'f16' else np.float32)
            call('ck_upload_param', self._h, name.encode(), arr.ctypes.data, arr.nbytes)

        with ThreadPoolExecutor(max_workers=max(1, threads)) as ex:
            list(ex.map(one, table))

    # -- frames -----------------------------------------------------------------
    def run_frame(self, warped_np, packed):
        """One policy frame (run_pinned2.py:1462-1565): uint8 [2,6,H,W] and
        f32 [524] in, flat f32 output vector out."""
        w = np.ascontiguousarray(warped_np, dtype=np.uint8)
        p = np.ascontiguousarray(packed, dtype=np.float32)
        s = self.spec
        if w.shape != (2, 6, s['img_h'], s['img_w']):
            raise ValueError(f'warped must be uint8 {(2, 6, s["img_h"], s["img_w"])}, got {w.shape}')
        if p.shape != self.PACKED.shape:
            raise ValueError(f'packed must be f32 {self.PACKED.shape}, got {p.shape}')
        self.PACKED[:] = p                   # PACKED[:] = packed (run_pinned2.py:1464)
        out = np.empty(self.n_out, np.float32)
        call('ck_run_frame', self._h, w.ctypes.data, p.ctypes.data, out.ctypes.data)
        return out

    def run_frame_nv12(self, frame, big_frame, tfm, big_tfm, packed):
        """One step of modeld's flow (compile_modeld.py:181-221): two NV12
        frames (flat uint8, the spec's "camera" geometry) and their f32 3x3
        inverse transforms are warped on device, then the frame runs as in
        run_frame.  Returns the flat f32 output vector."""
        cam = self.spec.get('camera')
        if not cam:
            raise ValueError('run_frame_nv12 needs a spec with a "camera" object')
        nb = _spec.nv12_bytes(cam)
        f = np.ascontiguousarray(frame, dtype=np.uint8).reshape(-1)
        bf = np.ascontiguousarray(big_frame, dtype=np.uint8).reshape(-1)
        if f.size != nb or bf.size != nb:
            raise ValueError(f'frames must be {nb} bytes of NV12, got {f.size} and {bf.size}')
        t = np.ascontiguousarray(tfm, dtype=np.float32)
        bt = np.ascontiguousarray(big_tfm, dtype=np.float32)
        if t.size != 9 or bt.size != 9:
            raise ValueError('transforms must be 3x3')
        p = np.ascontiguousarray(packed, dtype=np.float32)
        if p.shape != self.PACKED.shape:
            raise ValueError(f'packed must be f32 {self.PACKED.shape}, got {p.shape}')
        out = np.empty(self.n_out, np.float32)
        call('ck_run_frame_nv12', self._h, f.ctypes.data, bf.ctypes.data, nb, t.ctypes.data, bt.ctypes.data,
             p.ctypes.data, out.ctypes.data)
        return out

    def make_warped(self, val=128):
        """Constant frame pair (run_pinned2.py:1388-1389)."""
        s = self.spec
        return np.full((2, 6, s['img_h'], s['img_w']), val, np.uint8)

    def set_graph(self, on):
        call('ck_set_graph', self._h, 1 if on else 0)

    def graph_nodes(self):
        n = ctypes.c_size_t()
        call('ck_graph_nodes', self._h, ctypes.byref(n))
        return n.value

    def reset(self):
        call('ck_reset', self._h)

    def frame_launch(self):
        call('ck_frame_launch', self._h)

    def synchronize(self):
        call('ck_synchronize', self._h)

    def stream(self):
        s = ctypes.c_void_p()
        call('ck_stream', self._h, ctypes.byref(s))
        return s.value

    # -- plan / profiling ------------------------------------------------------
    def plan(self):
        n = ctypes.c_int()
        call('ck_plan_size', self._h, ctypes.byref(n))
        name = ctypes.create_string_buffer(128)
        kern = ctypes.create_string_buffer(128)
        fl, by = ctypes.c_double(), ctypes.c_double()
        out = []
        for i in range(n.value):
            call('ck_plan_entry', self._h, i, name, len(name), kern, len(kern), ctypes.byref(fl), ctypes.byref(by))
            out.append({'name': name.value.decode(), 'kernel': kern.value.decode(), 'flops': fl.value,
                        'bytes': by.value})
        return out

    def plan_index(self, name):
        for i, e in enumerate(self.plan()):
            if e['name'] == name:
                return i
        raise KeyError(name)

    def kernel_times(self):
        """One eager frame with per-launch event timing (KSYNC)."""
        plan = self.plan()
        ms = (ctypes.c_float * len(plan))()
        call('ck_kernel_times', self._h, ms, len(plan))
        for e, t in zip(plan, ms):
            e['ms'] = float(t)
        return plan

    def run_range(self, first, last):
        call('ck_run_range', self._h, int(first), int(last))

    def time_launches(self, indices, reps=1):
        """Elapsed ms of launching plan entries `indices` in order, `reps`
        times, between HIP events on the engine stream."""
        idx = (ctypes.c_int * len(indices))(*indices)
        ms = ctypes.c_float()
        call('ck_time_launches', self._h, idx, len(indices), int(reps), ctypes.byref(ms))
        return ms.value

    def time_in_frames(self, indices, frames=5):
        """Kernel time (ms) of plan entries `indices` inside `frames` whole
        eager frames, from each kernel's own start and end timestamps: the
        per-entry times per frame (a list) and their mean."""
        if not indices:
            raise ValueError('time_in_frames: no plan entries given')
        idx = (ctypes.c_int * len(indices))(*indices)
        per = (ctypes.c_float * len(indices))()
        mean = ctypes.c_float()
        call('ck_time_in_frames', self._h, idx, len(indices), int(frames), per, ctypes.byref(mean))
        return list(per), mean.value

    # -- tensors ----------------------------------------------------------------
    def tensor_ptr(self, name):
        p = ctypes.c_void_p()
        nb = ctypes.c_size_t()
        call('ck_tensor', self._h, name.encode(), ctypes.byref(p), ctypes.byref(nb))
        return p.value, nb.value

    def read(self, name, dtype, shape=None):
        _, nb = self.tensor_ptr(name)
        dtype = np.dtype(dtype)
        count = nb // dtype.itemsize if shape is None else int(np.prod(shape))
        out = np.empty(count, dtype)
        call('ck_read_tensor', self._h, name.encode(), out.ctypes.data, out.nbytes)
        return out if shape is None else out.reshape(shape)

    def write(self, name, arr):
        arr = np.ascontiguousarray(arr)
        call('ck_write_tensor', self._h, name.encode(), arr.ctypes.data, arr.nbytes)

    def parsed_outputs(self):
        """The Parser's output dictionary (parse_model_outputs.py:117-120) of
        the last frame, from the device decode that ends every frame."""
        from .parse import assemble
        self.synchronize()
        return assemble(self.read('decoded', np.float32), self.decoded_layout)

    # -- frame state (probe pre-state capture, cf. r62_probe.py:28-44) ------------
    def state_names(self):
        """[(name, nbytes, numpy dtype)] of every non-parameter tensor."""
        n = ctypes.c_int()
        call('ck_state_count', self._h, ctypes.byref(n))
        out = []
        name = ctypes.create_string_buffer(256)
        nb = ctypes.c_size_t()
        dt = ctypes.c_int()
        for i in range(n.value):
            call('ck_state_info', self._h, i, name, len(name), ctypes.byref(nb), ctypes.byref(dt))
            out.append((name.value.decode(), nb.value, _DT[dt.value]))
        return out

    def snapshot(self):
        """Host copies of the whole frame state: {name: 1-D array}."""
        self.synchronize()
        return {n: self.read(n, dt) for n, _, dt in self.state_names()}

    def restore(self, state):
        """Write a snapshot back (every tensor it holds)."""
        self.synchronize()
        for n, a in state.items():
            self.write(n, a)

    def state_hashes(self):
        """{name: 64-bit content hash} of every state tensor, whole tensor,
        computed on the device after the work already queued (ck_state_hashes)."""
        names = [n for n, _, _ in self.state_names()]
        out = (ctypes.c_uint64 * len(names))()
        call('ck_state_hashes', self._h, out, len(names))
        return dict(zip(names, (int(v) for v in out)))

    def fingerprints(self, frames=1, timed=True):
        """KSYNC with pre-state fingerprints (run_pinned2.py:1513-1557): `frames`
        eager frames launch by launch, each launch's pre-state hashed (every
        state tensor, ck_state_hashes) and, with `timed`, the launch timed
        alone between HIP events.  Returns a list with one row per launch,
        {'frame', 'index', 'name', 'kernel', 'ms', 'pre': {tensor: hash}},
        plus a last row (index = plan size) holding the state after the final
        launch.  The frames continue the engine's recurrent state."""
        plan = self.plan()
        rows = []
        for f in range(frames):
            for i, e in enumerate(plan):
                pre = self.state_hashes()
                ms = self.time_launches([i], 1) if timed else None
                if not timed:
                    self.run_range(i, i + 1)
                rows.append({'frame': f, 'index': i, 'name': e['name'], 'kernel': e['kernel'], 'ms': ms, 'pre': pre})
        rows.append({'frame': frames - 1, 'index': len(plan), 'name': '(end of frame)', 'kernel': '', 'ms': None,
                     'pre': self.state_hashes()})
        return rows


class Queues(Mapping):
    """The reference's `queues` dict (run_pinned2.py:1379-1386), read live
    from the device rings.

    The engine never shifts its queues: each is a ring indexed by the frame
    counter (csrc/pack.hip).  Reading a key rebuilds the reference's queue,
    oldest entry first, from the ring and the counter -- after N frames
    position j of a length-L queue holds the entry of frame N - L + j (zero
    for frames before the first), exactly what the reference's shift-by-one
    queues hold:
      img_q, big_img_q   uint8 (FS*(n_frames-1)+1, 6, H, W)
      feat_q             f32 (FS*feat_hist, 1, feat_len)
      desire_q           f32 (FS*desire_hist, 1, desire_len)
      packed_npy_inputs  the PACKED staging vector (desire | tc | action_t | prev_feat)
    Values are host copies taken at the time of the lookup.
    """

    _KEYS = ('img_q', 'big_img_q', 'feat_q', 'desire_q', 'packed_npy_inputs')

    def __init__(self, eng):
        self._eng = eng

    def __iter__(self):
        return iter(self._KEYS)

    def __len__(self):
        return len(self._KEYS)

    def frames(self):
        """Frames pushed since the last reset (the device frame counter)."""
        return int(self._eng.read('counter', np.uint32)[0])

    @staticmethod
    def _unroll(ring, n):
        """Reference order of a ring of L entries after n pushes."""
        L = ring.shape[0]
        out = np.zeros_like(ring)
        for j in range(L):
            f = n - L + j
            if f >= 0:
                out[j] = ring[f % L]
        return out

    def __getitem__(self, key):
        e, s = self._eng, self._eng.spec
        if key == 'packed_npy_inputs':
            return e.PACKED
        if key not in self._KEYS:
            raise KeyError(key)
        fs = s.get('frame_skip', 4)
        n = self.frames()
        if key in ('img_q', 'big_img_q'):
            slots = fs * (s.get('n_frames', 2) - 1) + 1
            ring = e.read('img_ring', np.uint8, (2, slots, 6, s['img_h'], s['img_w']))
            return self._unroll(ring[0 if key == 'img_q' else 1], n)
        if key == 'feat_q':
            ring = e.read('feat_ring', np.float32, (fs * s['feat_hist'], 1, s['feat_len']))
            return self._unroll(ring, n)
        ring = e.read('desire_ring', np.float32, (fs * s['desire_hist'], 1, s['desire_len']))
        return self._unroll(ring, n)


def load(spec='big_driving_1b', **kw):
    """The reference's exec-prefix namespace (run_pinned2.py:1346-1572;
    video_demo.py:25): run_frame, out_slices, img, make_warped, queues,
    PACKED, plus the engine."""
    eng = Engine(spec, **kw)
    return types.SimpleNamespace(run_frame=eng.run_frame, out_slices=eng.out_slices, img=eng.img,
                                 make_warped=eng.make_warped, queues=Queues(eng), PACKED=eng.PACKED, engine=eng)
