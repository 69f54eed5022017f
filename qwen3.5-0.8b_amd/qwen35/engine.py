"""ctypes host over libqwen35.so (include/q35.h)."""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

VOCAB = 248320
HIDDEN = 1024
EOS_IDS = (248046, 248044)       # speccheck/specimpl.py:38-40

_PKG = Path(__file__).resolve().parents[1]
_LIB = None


class EngineError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"q35 error {code}: {msg}")
        self.code = code


def lib_path() -> Path:
    return _PKG / "libqwen35.so"


class _Config(C.Structure):
    _fields_ = [("device", C.c_int), ("max_rows", C.c_int), ("max_ctx", C.c_int),
                ("use_graph", C.c_int)]


_SIGS = {
    "q35_last_error": ([], C.c_char_p),
    "q35_create": ([C.POINTER(_Config), C.POINTER(C.c_void_p)], C.c_int),
    "q35_destroy": ([C.c_void_p], C.c_int),
    "q35_init_random": ([C.c_void_p, C.c_uint64], C.c_int),
    "q35_load_tensor": ([C.c_void_p, C.c_char_p, C.c_void_p, C.c_size_t], C.c_int),
    "q35_read_tensor": ([C.c_void_p, C.c_char_p, C.c_void_p, C.c_size_t], C.c_int),
    "q35_load_safetensors": ([C.c_void_p, C.c_void_p, C.c_size_t, C.POINTER(C.c_int32), C.POINTER(C.c_int32)],
                             C.c_int),
    "q35_safetensors_scan": ([C.c_void_p, C.c_size_t, C.POINTER(C.c_int32), C.POINTER(C.c_int32)], C.c_int),
    "q35_state_alloc": ([C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_void_p)], C.c_int),
    "q35_state_free": ([C.c_void_p, C.c_void_p], C.c_int),
    "q35_state_reset": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int], C.c_int),
    "q35_state_seed": ([C.c_void_p, C.c_void_p, C.c_uint64, C.c_int], C.c_int),
    "q35_state_prefix_len": ([C.c_void_p, C.c_void_p, C.c_int, C.POINTER(C.c_int32)], C.c_int),
    "q35_state_read": ([C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_size_t], C.c_int),
    "q35_state_write": ([C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_size_t], C.c_int),
    "q35_state_copy_lane": ([C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int], C.c_int),
    "q35_state_snapshot": ([C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_size_t, C.POINTER(C.c_size_t)],
                           C.c_int),
    "q35_state_restore": ([C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_size_t], C.c_int),
    "q35_prefill": ([C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.POINTER(C.c_int32), C.c_void_p], C.c_int),
    "q35_prefill_all": ([C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p,
                         C.c_void_p], C.c_int),
    "q35_decode_step": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p], C.c_int),
    "q35_mtp_draft": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int,
                       C.c_void_p, C.c_void_p, C.c_void_p], C.c_int),
    "q35_mtp_round": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_void_p,
                       C.c_void_p, C.c_void_p], C.c_int),
    "q35_mtp_round_stop": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int32,
                            C.c_void_p, C.c_void_p, C.c_void_p], C.c_int),
    "q35_mtp_policy_create": ([C.c_int, C.c_double, C.c_double, C.POINTER(C.c_void_p)], C.c_int),
    "q35_mtp_policy_free": ([C.c_void_p], C.c_int),
    "q35_mtp_policy_k": ([C.c_void_p, C.POINTER(C.c_int32)], C.c_int),
    "q35_mtp_policy_note": ([C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.POINTER(C.c_double)], C.c_int),
    "q35_mtp_adaptive_step": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int32,
                               C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p], C.c_int),
    "q35_op_tile_weight": ([C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p], C.c_int),
    "q35_op_gemm": ([C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_void_p], C.c_int),
    "q35_op_gdn_step": ([C.c_void_p] * 8 + [C.c_int], C.c_int),
    "q35_op_gdn_step_noalloc": ([C.c_void_p] * 8 + [C.c_int], C.c_int),
    "q35_op_gdn_step_norm": ([C.c_void_p] * 10 + [C.c_int, C.c_int], C.c_int),
    "q35_op_gemm_a": ([C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_void_p,
                       C.c_int, C.c_void_p, C.c_int, C.c_void_p], C.c_int),
    "q35_prefill_lanes": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p,
                           C.c_void_p], C.c_int),
    "q35_mtp_verify": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_int32,
                        C.c_void_p, C.c_void_p, C.c_void_p], C.c_int),
    "q35_op_attn_decode": ([C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_int]
                           + [C.c_void_p] * 4 + [C.c_int], C.c_int),
    "q35_op_lm_head_argmax": ([C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p], C.c_int),
    "q35_sync": ([C.c_void_p], C.c_int),
    "q35_kprof_read": ([C.c_void_p, C.POINTER(C.c_float), C.POINTER(C.c_int)], C.c_int),
    "q35_set_option": ([C.c_void_p, C.c_char_p, C.c_int], C.c_int),
    "q35_read_scratch": ([C.c_void_p, C.c_char_p, C.c_void_p, C.c_size_t], C.c_int),
    "q35_timer_begin": ([C.c_void_p], C.c_int),
    "q35_timer_end": ([C.c_void_p, C.POINTER(C.c_float)], C.c_int),
}


def load_library():
    """Loads libqwen35.so (raises if it was not built: there is no fallback path)."""
    global _LIB
    if _LIB is None:
        p = lib_path()
        if not p.exists():
            raise EngineError(-3, f"{p} is missing; build it with qwen3.5-0.8b_amd/build.py")
        L = C.CDLL(str(p))
        for name, (args, res) in _SIGS.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = res
        _LIB = L
    return _LIB


def _ck(rc: int):
    if rc != 0:
        raise EngineError(rc, load_library().q35_last_error().decode())


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def safetensors_scan(data: bytes | np.ndarray) -> tuple[int, int]:
    """(tensors, vision tensors) of a .safetensors container, validated by the library's parser
    without an engine or a GPU (q35_safetensors_scan); raises EngineError on a malformed file."""
    b = np.frombuffer(data, dtype=np.uint8) if isinstance(data, (bytes, bytearray)) else data
    nt, nv = C.c_int32(), C.c_int32()
    _ck(load_library().q35_safetensors_scan(C.c_void_p(b.ctypes.data) if b.size else None, b.size,
                                            C.byref(nt), C.byref(nv)))
    return nt.value, nv.value


class Engine:
    """Weights + scratch + stream (WeightStore / DecodeScratch of the reference)."""

    def __init__(self, max_rows: int = 256, max_ctx: int = 4352, device: int = 0, seed: int | None = 0,
                 use_graph: bool = False):
        L = load_library()
        cfg = _Config(device, max_rows, max_ctx, int(use_graph))
        h = C.c_void_p()
        _ck(L.q35_create(C.byref(cfg), C.byref(h)))
        self.h = h
        self.max_rows = max_rows
        self.max_ctx = max_ctx
        if seed is not None:
            self.init_random(seed)

    def init_random(self, seed: int):
        _ck(load_library().q35_init_random(self.h, seed))

    def load_tensor(self, name: str, bits: np.ndarray):
        b = np.ascontiguousarray(bits, dtype=np.uint16)
        _ck(load_library().q35_load_tensor(self.h, name.encode(), _p(b), b.size))

    def load_checkpoint(self, model_dir) -> tuple[int, int]:
        """Weights from the checkpoint directory's .safetensors file, as specimpl.Weights
        (speccheck/specimpl.py:70-86) loads it: the first *.safetensors found, vision tensors
        skipped, everything cast to bf16. The file is memory-mapped and parsed by the library
        (q35_load_safetensors). Returns (loaded, skipped) = (335, 153)."""
        path = next(Path(model_dir).glob("*.safetensors"))
        buf = np.memmap(path, dtype=np.uint8, mode="r")
        loaded, skipped = C.c_int32(), C.c_int32()
        try:
            _ck(load_library().q35_load_safetensors(self.h, C.c_void_p(buf.ctypes.data), buf.size,
                                                    C.byref(loaded), C.byref(skipped)))
        finally:
            del buf
        return loaded.value, skipped.value

    def read_tensor(self, name: str, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.uint16)
        _ck(load_library().q35_read_tensor(self.h, name.encode(), _p(out), n))
        return out

    def set_option(self, name: str, value: int):
        _ck(load_library().q35_set_option(self.h, name.encode(), int(value)))

    def read_scratch(self, name: str, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        _ck(load_library().q35_read_scratch(self.h, name.encode(), _p(out), out.nbytes))
        return out

    def kprof_read(self):
        ms, n = C.c_float(), C.c_int()
        _ck(load_library().q35_kprof_read(self.h, C.byref(ms), C.byref(n)))
        return ms.value, n.value

    def sync(self):
        _ck(load_library().q35_sync(self.h))

    def close(self):
        if self.h:
            load_library().q35_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # per-op (device pointers as ints, e.g. torch tensor.data_ptr())
    def op_tile_weight(self, w_ptr: int, N: int, K: int, wt_ptr: int):
        _ck(load_library().q35_op_tile_weight(self.h, C.c_void_p(w_ptr), N, K, C.c_void_p(wt_ptr)))

    def op_gemm(self, wt_ptr: int, N: int, K: int, x_ptr: int, M: int, y_ptr: int):
        _ck(load_library().q35_op_gemm(self.h, C.c_void_p(wt_ptr), N, K, C.c_void_p(x_ptr), M, C.c_void_p(y_ptr)))

    def op_gdn_step(self, proj: int, conv_w: int, A_log: int, dt_bias: int, S2: int, W2: int, o: int, B: int):
        _ck(load_library().q35_op_gdn_step(self.h, *[C.c_void_p(p) for p in (proj, conv_w, A_log, dt_bias, S2, W2, o)], B))

    def op_gdn_step_noalloc(self, proj: int, conv_w: int, A_log: int, dt_bias: int, S2: int, W2: int, o: int, B: int):
        """The allocation-free GDN step (asynchronous on the engine stream: sync() waits)."""
        _ck(load_library().q35_op_gdn_step_noalloc(self.h, *[C.c_void_p(p) for p in (proj, conv_w, A_log, dt_bias,
                                                                                       S2, W2, o)], B))

    def op_gdn_step_norm(self, proj: int, conv_w: int, A_log: int, dt_bias: int, gnorm: int, S2: int, W2: int,
                         o: int, y: int, B: int, form: int = 0):
        _ck(load_library().q35_op_gdn_step_norm(
            self.h, *[C.c_void_p(p) for p in (proj, conv_w, A_log, dt_bias, gnorm, S2, W2, o, y)], B, form))

    def op_gemm_a(self, wt_ptr: int, N: int, K: int, amode: int, x_ptr: int, ldx: int, x2_ptr: int, ldx2: int,
                  aux_ptr: int, M: int, y_ptr: int):
        _ck(load_library().q35_op_gemm_a(self.h, C.c_void_p(wt_ptr), N, K, amode, C.c_void_p(x_ptr), ldx,
                                         C.c_void_p(x2_ptr) if x2_ptr else None, ldx2,
                                         C.c_void_p(aux_ptr) if aux_ptr else None, M, C.c_void_p(y_ptr)))

    def op_attn_decode(self, state: "State", layer: int, lanes, pos, T: int, proj: int, q_norm: int, k_norm: int,
                       out: int, form: int = 0):
        """One attention layer on `state`'s cache (q35_op_attn_decode): rows of lane lanes[i] at
        positions pos[i] .. pos[i] + T - 1 (None: the lanes' prefix lengths)."""
        la = _i32(lanes)
        pa = None if pos is None else _i32(pos)
        _ck(load_library().q35_op_attn_decode(self.h, state.h, layer, _p(la), None if pa is None else _p(pa), la.size,
                                              T, *[C.c_void_p(p) for p in (proj, q_norm, k_norm, out)], form))

    def op_lm_head_argmax(self, x_ptr: int, M: int, tok_ptr: int, logits_ptr: int = 0):
        _ck(load_library().q35_op_lm_head_argmax(self.h, C.c_void_p(x_ptr), M, C.c_void_p(tok_ptr),
                                                 C.c_void_p(logits_ptr) if logits_ptr else None))

    def timer_begin(self):
        _ck(load_library().q35_timer_begin(self.h))

    def timer_end(self) -> float:
        ms = C.c_float()
        _ck(load_library().q35_timer_end(self.h, C.byref(ms)))
        return ms.value


# Round cost in plain decode steps of an MTP round at depth k, measured on one MI355X at batch 1,
# ctx 4,096 (bench.py `mtp_k2.b1_k1` / `mtp_k2.b1` round_cost_steps: a k = 1 round 1.552 steps, a
# k = 2 round 1.920). The reference bills its own gfx1151 rounds at 1.58 / 1.90
# (engine/mtp_adaptive.h:54-68); a policy on this engine uses these instead.
MI355X_ROUND_COST = {1: 1.552, 2: 1.920}


class MtpPolicy:
    """Adaptive speculation depth of one request (mtpadapt::Tracker, engine/mtp_adaptive.h):
    k = 2 -> 1 -> 0 (plain) from the request's own rounds; costs <= 0 take the reference's
    round / step ratios (1.58 at k = 1, 1.90 at k = 2)."""

    def __init__(self, start_k: int = 2, cost_k1: float = 0.0, cost_k2: float = 0.0):
        h = C.c_void_p()
        _ck(load_library().q35_mtp_policy_create(start_k, cost_k1, cost_k2, C.byref(h)))
        self.h = h

    @property
    def k(self) -> int:
        v = C.c_int32()
        _ck(load_library().q35_mtp_policy_k(self.h, C.byref(v)))
        return v.value

    def note(self, k_round: int, emitted: int):
        """Feed one round; returns (change or None, est) with change = (from, to, rounds seen)."""
        ch = np.full(3, -1, np.int32)
        est = C.c_double()
        _ck(load_library().q35_mtp_policy_note(self.h, k_round, emitted, _p(ch), C.byref(est)))
        return (tuple(int(x) for x in ch) if ch[0] >= 0 else None), est.value

    def close(self):
        if self.h:
            load_library().q35_mtp_policy_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class State:
    """`lanes` independent requests (RequestState, engine/state.h:83-116)."""

    def __init__(self, eng: Engine, lanes: int = 1, cap: int = 4352, mtp_k: int = 0, mtp_cap: int = 0):
        self.eng = eng
        self.lanes, self.cap, self.mtp_k, self.mtp_cap = lanes, cap, mtp_k, mtp_cap
        h = C.c_void_p()
        _ck(load_library().q35_state_alloc(eng.h, lanes, cap, mtp_k, mtp_cap, C.byref(h)))
        self.h = h

    def reset(self, lanes=None):
        if lanes is None:
            _ck(load_library().q35_state_reset(self.eng.h, self.h, None, 0))
        else:
            a = _i32(lanes)
            _ck(load_library().q35_state_reset(self.eng.h, self.h, _p(a), a.size))

    def seed(self, seed: int, prefix_len: int):
        _ck(load_library().q35_state_seed(self.eng.h, self.h, seed, prefix_len))

    def prefix_len(self, lane: int = 0) -> int:
        v = C.c_int32()
        _ck(load_library().q35_state_prefix_len(self.eng.h, self.h, lane, C.byref(v)))
        return v.value

    def read(self, lane: int, which: str, n_slots: int = 0) -> np.ndarray:
        shapes = {"S": ((18, 16, 128, 128), np.float32, 0), "win": ((18, 3, 6144), np.float32, 1),
                  "k": ((6, 2, n_slots, 256), np.uint16, 2), "v": ((6, 2, n_slots, 256), np.uint16, 3),
                  "mk": ((2, n_slots, 256), np.uint16, 4), "mv": ((2, n_slots, 256), np.uint16, 5)}
        shape, dt, w = shapes[which]
        out = np.empty(shape, dtype=dt)
        _ck(load_library().q35_state_read(self.eng.h, self.h, lane, w, n_slots, _p(out), out.nbytes))
        return out

    def write(self, lane: int, which: str, arr: np.ndarray, n_slots: int = 0):
        w = {"S": 0, "win": 1, "k": 2, "v": 3, "mk": 4, "mv": 5}[which]
        a = np.ascontiguousarray(arr)
        _ck(load_library().q35_state_write(self.eng.h, self.h, lane, w, n_slots, _p(a), a.nbytes))

    def close(self):
        if self.h:
            load_library().q35_state_free(self.eng.h, self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- engine calls over this state
    def copy_lane(self, lane: int, dst: "State", dst_lane: int):
        """Fork this lane's whole tuple (S, conv window, KV[0, P), MTP cache, last hidden row,
        P) into dst's lane, device to device: prefix reuse (specification/08-state-management.md
        §08.3)."""
        _ck(load_library().q35_state_copy_lane(self.eng.h, self.h, lane, dst.h, dst_lane))

    def snapshot(self, lane: int) -> np.ndarray:
        """The lane's tuple as one contiguous host blob (preempt, §08.4)."""
        n = C.c_size_t()
        _ck(load_library().q35_state_snapshot(self.eng.h, self.h, lane, None, 0, C.byref(n)))
        buf = np.empty(n.value, np.uint8)
        _ck(load_library().q35_state_snapshot(self.eng.h, self.h, lane, _p(buf), buf.size, C.byref(n)))
        return buf

    def restore(self, lane: int, blob: np.ndarray):
        """Write a snapshot back into a lane (resume, §08.4)."""
        b = np.ascontiguousarray(blob, dtype=np.uint8)
        _ck(load_library().q35_state_restore(self.eng.h, self.h, lane, _p(b), b.size))

    def prefill(self, lane: int, ids, logits: bool = False):
        ids = _i32(ids)
        y0 = C.c_int32()
        lg = np.empty(VOCAB, np.float32) if logits else None
        _ck(load_library().q35_prefill(self.eng.h, self.h, lane, _p(ids), ids.size, C.byref(y0),
                                       _p(lg) if logits else None))
        return (y0.value, lg) if logits else y0.value

    def prefill_lanes(self, prompts, lanes=None, logits: bool = False):
        """Prompts of several lanes in shared body passes (q35_prefill_lanes): prompts[i] goes to
        lane lanes[i] (i when None); returns the greedy ids after each prompt (and their logits)."""
        ids = _i32(np.concatenate([np.asarray(p, np.int32) for p in prompts]))
        lens = _i32([len(p) for p in prompts])
        n = lens.size
        ln = _i32(lanes) if lanes is not None else None
        y0 = np.zeros(n, np.int32)
        lg = np.empty((n, VOCAB), np.float32) if logits else None
        _ck(load_library().q35_prefill_lanes(self.eng.h, self.h, _p(ln) if ln is not None else None, n, _p(ids),
                                             _p(lens), _p(y0), _p(lg) if logits else None))
        return (y0, lg) if logits else y0

    def prefill_all(self, lane: int, ids, logits: bool = False):
        """The prompt with every row priced (PrefillLogits::kAll, engine/prefill.h:46-58): per-row
        greedy ids and top logit values, and optionally every row's logits [n][248320]."""
        ids = _i32(ids)
        n = ids.size
        samp = np.empty(n, np.int32)
        top = np.empty(n, np.float32)
        lg = np.empty((n, VOCAB), np.float32) if logits else None
        _ck(load_library().q35_prefill_all(self.eng.h, self.h, lane, _p(ids), n, _p(samp), _p(top),
                                           _p(lg) if logits else None))
        return (samp, top, lg) if logits else (samp, top)

    def decode_step(self, tokens, lanes=None, logits: bool = False):
        t = _i32(tokens)
        n = t.size
        ln = _i32(lanes) if lanes is not None else None
        out = np.empty(n, np.int32)
        lg = np.empty((n, VOCAB), np.float32) if logits else None
        _ck(load_library().q35_decode_step(self.eng.h, self.h, _p(ln) if ln is not None else None, n,
                                           _p(t), _p(out), _p(lg) if logits else None))
        return (out, lg) if logits else out

    def mtp_draft(self, y, pos, step: int, lanes=None, logits: bool = False):
        y, pos = _i32(y), _i32(pos)
        n = y.size
        ln = _i32(lanes) if lanes is not None else None
        out = np.empty(n, np.int32)
        xd = np.empty((n, HIDDEN), np.uint16)
        lg = np.empty((n, VOCAB), np.float32) if logits else None
        _ck(load_library().q35_mtp_draft(self.eng.h, self.h, _p(ln) if ln is not None else None, n, _p(y),
                                         _p(pos), step, _p(out), _p(xd), _p(lg) if logits else None))
        return out, xd, lg

    def mtp_verify(self, cur, drafts, lanes=None, stats: np.ndarray | None = None, stop: int = -1):
        """The verify half of a round on the caller's drafts [n][k] (mtpaccept::accept_round's
        candidates); returns each lane's emitted tokens."""
        c = _i32(cur)
        d = np.ascontiguousarray(np.asarray(drafts, np.int32).reshape(c.size, -1))
        n, k = d.shape
        ln = _i32(lanes) if lanes is not None else None
        emit = np.zeros((n, k + 1), np.int32)
        ne = np.zeros(n, np.int32)
        st = stats if stats is not None else np.zeros(4, np.int64)
        _ck(load_library().q35_mtp_verify(self.eng.h, self.h, _p(ln) if ln is not None else None, n, _p(c), k,
                                          _p(d), stop, _p(emit), _p(ne), _p(st)))
        return [list(emit[i, :ne[i]]) for i in range(n)]

    def mtp_round(self, cur, k: int, lanes=None, stats: np.ndarray | None = None, stop: int = -1):
        """One speculative round per lane; stop >= 0 applies the session's stop cut (an
        accepted draft equal to it ends the lane's emits and stays pending)."""
        c = _i32(cur)
        n = c.size
        ln = _i32(lanes) if lanes is not None else None
        emit = np.zeros((n, k + 1), np.int32)
        ne = np.zeros(n, np.int32)
        st = stats if stats is not None else np.zeros(4, np.int64)
        _ck(load_library().q35_mtp_round_stop(self.eng.h, self.h, _p(ln) if ln is not None else None, n, _p(c),
                                              k, stop, _p(emit), _p(ne), _p(st)))
        return [list(emit[i, :ne[i]]) for i in range(n)]


    def mtp_adaptive_step(self, cur, policies, lanes=None, stop: int = -1, stats: np.ndarray | None = None):
        """One turn of the lanes, each at its policy's depth (q35_mtp_adaptive_step): returns the
        emitted tokens per lane and the depth each lane ran at (0 = a plain step)."""
        c = _i32(cur)
        n = c.size
        assert len(policies) == n
        ln = _i32(lanes) if lanes is not None else None
        pol = (C.c_void_p * n)(*[p.h.value for p in policies])
        emit = np.full((n, 3), -1, np.int32)
        ne = np.zeros(n, np.int32)
        dep = np.zeros(n, np.int32)
        st = stats if stats is not None else np.zeros(4, np.int64)
        _ck(load_library().q35_mtp_adaptive_step(self.eng.h, self.h, _p(ln) if ln is not None else None, n, _p(c),
                                                 C.cast(pol, C.c_void_p), stop, _p(emit), _p(ne), _p(dep), _p(st)))
        return [list(emit[i, :ne[i]]) for i in range(n)], dep


class Forward:
    """One lane driven like specimpl.Forward (prefill / decode / greedy)."""

    def __init__(self, eng: Engine, state: State | None = None, lane: int = 0, cap: int = 4352):
        self.eng = eng
        self.state = state if state is not None else State(eng, 1, cap)
        self.lane = lane

    @property
    def P(self) -> int:
        return self.state.prefix_len(self.lane)

    def reset(self):
        self.state.reset([self.lane])

    def prefill(self, ids, logits: bool = False):
        return self.state.prefill(self.lane, ids, logits)

    def decode(self, tok: int, logits: bool = False):
        r = self.state.decode_step([tok], [self.lane], logits)
        return (int(r[0][0]), r[1][0]) if logits else int(r[0])

    def greedy(self, ids, steps: int, stop_on_eos: bool = True, logits_out=None):
        """specimpl.py:496-517: first token from the prompt, then `steps` decodes."""
        want = logits_out is not None
        r = self.prefill(ids, want)
        if want:
            tok, lg = r
            logits_out.append(lg)
        else:
            tok = r
        out = [tok]
        for _ in range(steps):
            if stop_on_eos and out[-1] in EOS_IDS:
                break
            r = self.decode(out[-1], want)
            if want:
                tok, lg = r
                logits_out.append(lg)
            else:
                tok = r
            out.append(tok)
        return out


def greedy_mtp(f: Forward, ids, steps: int, k: int = 2, stop_on_eos: bool = True,
               policy: "MtpPolicy | None" = None):
    """speccheck/mtp.py:97-179 with the batched verify and rollback done in the engine; with a
    policy, each round's depth is the policy's (engine/mtp_adaptive.h), 0 meaning a plain step."""
    assert f.state.mtp_k >= k
    stats = np.zeros(4, np.int64)
    t = f.prefill(ids)
    out = [t]
    while len(out) < steps + 1 and not (stop_on_eos and out[-1] in EOS_IDS):
        if policy is not None:
            em = f.state.mtp_adaptive_step([out[-1]], [policy], [f.lane], stats=stats)[0][0]
        else:
            em = f.state.mtp_round([out[-1]], k, [f.lane], stats)[0]
        out.extend(int(x) for x in em)
    return out, dict(drafted=int(stats[0]), accepted=int(stats[1]), bonus=int(stats[2]),
                     verify_tokens=int(stats[3]), target_forwards=int(stats[2]) + 1)
