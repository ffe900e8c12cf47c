"""Linear-path mirror of the reference's decoder.py on libtyphoon_linear.so.

The reference's Decoder (decoder.py:182-523) quantizes every projection at
load with the library's w8a32_quantize (:248-260), keeps the int8/scale arrays
alive (:215, :259), concatenates Q||K||V and gate||up for prefill (:290-302),
registers the pointers with the C decoder (:304-317), and per generated token
computes the lm_head logits with w8a32_linear(batch=1) after a numpy final
RMSNorm (:443-460), then samples (:462-477).

This module keeps those steps with the same names, argument meaning and
error behaviour, on the MI355X library:
  * load_decoder_lib() binds w8a32_quantize / w8a32_linear with the
    reference's argtypes (decoder.py:145-157) plus tl_last_error;
  * Decoder quantizes on the GPU (w8a32_quantize packs the HBM tiles in the
    same pass and keeps them for the returned host arrays), packs the fused
    matrices, and registers every quantized matrix with tl_register_weights
    (only the fused copies upload anything there); with the layer norms it
    hands the layer, fused matrices included, to the device loop through
    decoder_set_layer_weights_v32, as the reference does (:304-317);
  * save_cache() / from_cache() write and read a packed-weight cache file,
    so a later load copies the HBM tiles back with no quantization;
  * project() runs one projection through w8a32_linear with the reference's
    batch-dependent numerics; get_logits() / sample() are _get_logits and the
    greedy branch of _sample.

With the layer norms given (random_layer_weights(norms=True) or real
weights), the Decoder also builds the device-resident layer loop through the
reference's decoder C ABI (decoder_set_layer_weights_v32, decoder_decode_step:
kernel/decoder.c:300-526): step() is the reference's Decoder.step, and
generate_greedy() runs the greedy decode loop on the GPU.
"""
from __future__ import annotations

import ctypes
from typing import Dict, List, Mapping, Optional

import numpy as np

from . import linear as _lin

# Qwen3-VL 2B constants (reference decoder.py:28-38)
HIDDEN_DIM = 2048
KV_DIM = 1024
FFN_DIM = 6144
NUM_Q_HEADS = 16
NUM_KV_HEADS = 8
HEAD_DIM = 128
NUM_LAYERS = 28
MAX_SEQ_LEN = 2048
TILE_M = 128
QKV_DIM = HIDDEN_DIM + 2 * KV_DIM      # 4096
GATE_UP_DIM = 2 * FFN_DIM              # 12288
VOCAB = 151936
RMS_EPS = 1e-6

PROJECTIONS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


def _np_ptr(arr: np.ndarray, ctype=ctypes.c_float):
    return arr.ctypes.data_as(ctypes.POINTER(ctype))


def load_decoder_lib() -> ctypes.CDLL:
    """Load the MI355X library with the reference's linear-path argtypes."""
    lib = _lin.load_library()
    _i8p = ctypes.POINTER(ctypes.c_int8)
    _f32p = ctypes.POINTER(ctypes.c_float)
    lib.w8a32_quantize.restype = None
    lib.w8a32_quantize.argtypes = [_f32p, _i8p, _f32p, ctypes.c_int, ctypes.c_int]
    lib.w8a32_linear.restype = None
    lib.w8a32_linear.argtypes = [_f32p, _i8p, _f32p, _f32p, _f32p, _f32p,
                                 ctypes.c_int, ctypes.c_int, ctypes.c_int]
    return lib


def qwen3vl_shapes(num_layers: int = NUM_LAYERS, vocab: int = VOCAB) -> Dict[str, tuple]:
    """(rows, cols) of every linear weight of the Qwen3-VL-2B text decoder."""
    per_layer = {"q_proj": (HIDDEN_DIM, HIDDEN_DIM), "k_proj": (KV_DIM, HIDDEN_DIM),
                 "v_proj": (KV_DIM, HIDDEN_DIM), "o_proj": (HIDDEN_DIM, HIDDEN_DIM),
                 "gate_proj": (FFN_DIM, HIDDEN_DIM), "up_proj": (FFN_DIM, HIDDEN_DIM),
                 "down_proj": (HIDDEN_DIM, FFN_DIM)}
    out = {f"layers.{l}.{k}": v for l in range(num_layers) for k, v in per_layer.items()}
    out["lm_head"] = (vocab, HIDDEN_DIM)
    return out


NORMS = ("input_ln", "post_attn_ln", "q_norm", "k_norm")
MROPE_SECTIONS = (24, 20, 20)           # reference decoder.py:40
MROPE_THETA_BASE = (5000000.0,) * 3     # reference decoder.py:41


def random_layer_weights(rng: np.random.Generator, hidden: int = HIDDEN_DIM, kv: int = KV_DIM,
                         ffn: int = FFN_DIM, std: float = 0.02, norms: bool = False) -> Dict[str, np.ndarray]:
    """Random-init fp32 weights of one layer's seven projections (and, with
    norms=True, its RMSNorm weights: input_ln / post_attn_ln [hidden],
    q_norm / k_norm [128], around 1)."""
    shapes = {"q_proj": (hidden, hidden), "k_proj": (kv, hidden), "v_proj": (kv, hidden),
              "o_proj": (hidden, hidden), "gate_proj": (ffn, hidden), "up_proj": (ffn, hidden),
              "down_proj": (hidden, ffn)}
    out = {k: (rng.standard_normal(s, dtype=np.float32) * np.float32(std)) for k, s in shapes.items()}
    if norms:
        for k, n in (("input_ln", hidden), ("post_attn_ln", hidden), ("q_norm", HEAD_DIM), ("k_norm", HEAD_DIM)):
            out[k] = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    return out


class Decoder:
    """Quantized linear layers of the text decoder, resident in HBM.

    layers:      sequence of mappings name -> fp32 [out, in] array for the seven
                 projections of each layer (PROJECTIONS)
    lm_head:     fp32 [vocab, hidden] (optional)
    final_norm:  fp32 [hidden] RMSNorm weight (optional)
    """

    def __init__(self, layers: List[Mapping[str, np.ndarray]], lib: Optional[ctypes.CDLL] = None,
                 lm_head: Optional[np.ndarray] = None, final_norm: Optional[np.ndarray] = None,
                 verbose: bool = False, max_seq: int = MAX_SEQ_LEN):
        self._lib = lib or load_decoder_lib()
        self._weight_store: list = []          # keep numpy arrays alive (reference :215)
        self.layers: List[Dict[str, tuple]] = []
        self._max_seq = max_seq
        self._c_model = self._c_cache = self._c_scratch = None   # device loop, built with the first norms
        for l_idx, layer in enumerate(layers):
            self._register_layer(l_idx, layer)
            if verbose and ((l_idx + 1) % 7 == 0 or l_idx == len(layers) - 1):
                print(f"\r[Decoder] Layer {l_idx + 1}/{len(layers)} ...", end="", flush=True)
        if verbose:
            print("\n[Decoder] Weights loaded.", flush=True)
        self._final_norm_w = None if final_norm is None else np.ascontiguousarray(final_norm, np.float32)
        self._lm_head_w = None
        if lm_head is not None:
            q, s = self._quantize_and_keep(lm_head)
            self._lm_head_w, self._lm_head_s = q, s
            self._lm_head_M, self._lm_head_K = q.shape
            self._lm_head_scratch = np.empty((TILE_M, self._lm_head_K), dtype=np.float32)
            self._weight_store.append(self._lm_head_scratch)
            self._register(q, s)
            self._logits_buf = np.empty(self._lm_head_M, dtype=np.float32)

    # -- packed-weight cache file ---------------------------------------------
    def _matrices(self):
        for l_idx, entry in enumerate(self.layers):
            for name, (w, s) in entry.items():
                yield f"layers.{l_idx}.{name}", w, s
        if self._lm_head_w is not None:
            yield "lm_head", self._lm_head_w, self._lm_head_s

    def save_cache(self, path: str) -> None:
        """Write every quantized matrix (the seven projections and the fused
        Q||K||V and gate||up of each layer, then the lm_head) as the records
        of one packed-weight cache file, named layers.<l>.<projection> and
        lm_head.  The file replaces any existing one."""
        first = True
        for name, w, s in self._matrices():
            W = _lin.DeviceWeights.from_codes(w, s)
            try:
                W.save(path, name, append=not first)
            finally:
                W.close()
            first = False

    @classmethod
    def from_cache(cls, path: str, lib: Optional[ctypes.CDLL] = None,
                   final_norm: Optional[np.ndarray] = None) -> "Decoder":
        """A Decoder whose quantized matrices come from a packed-weight cache
        file (save_cache) instead of fp32 weights: each record is copied into
        HBM as it is, its codes and scales are exported to host arrays (the
        arrays the reference keeps in _weight_store), and the device copy is
        handed to the host-pointer registry for those arrays, so no matrix is
        quantized, packed or uploaded a second time."""
        self = cls.__new__(cls)
        self._lib = lib or load_decoder_lib()
        self._weight_store = []
        self.layers = []
        self._max_seq = MAX_SEQ_LEN
        self._c_model = self._c_cache = self._c_scratch = None
        names = _lin.cache_list(path)
        n_layers = 1 + max((int(n.split(".")[1]) for n in names if n.startswith("layers.")), default=-1)
        for l_idx in range(n_layers):
            entry = {}
            for name in PROJECTIONS + ("qkv_proj", "gate_up_proj"):
                entry[name] = self._load_record(path, f"layers.{l_idx}.{name}")
            self.layers.append(entry)
        self._final_norm_w = None if final_norm is None else np.ascontiguousarray(final_norm, np.float32)
        self._lm_head_w = None
        if "lm_head" in names:
            q, s = self._load_record(path, "lm_head")
            self._lm_head_w, self._lm_head_s = q, s
            self._lm_head_M, self._lm_head_K = q.shape
            self._lm_head_scratch = np.empty((TILE_M, self._lm_head_K), dtype=np.float32)
            self._weight_store.append(self._lm_head_scratch)
            self._logits_buf = np.empty(self._lm_head_M, dtype=np.float32)
        return self

    def _load_record(self, path: str, name: str):
        W = _lin.DeviceWeights.load(path, name)
        try:
            codes, scales = W.export()
            W.adopt_into_registry(codes, scales)
        finally:
            W.close()
        self._weight_store.extend([codes, scales])
        return codes, scales

    # -- weight quantization helpers (reference :248-317) -------------------
    def _quantize_and_keep(self, w_fp32: np.ndarray):
        M, K = w_fp32.shape
        w_packed = np.empty((M, K), dtype=np.int8)
        scales = np.empty(M, dtype=np.float32)
        w_fp32_c = np.ascontiguousarray(w_fp32, dtype=np.float32)
        self._lib.w8a32_quantize(_np_ptr(w_fp32_c), _np_ptr(w_packed, ctypes.c_int8), _np_ptr(scales),
                                 ctypes.c_int(M), ctypes.c_int(K))
        _lin.check(self._lib, "w8a32_quantize")
        self._weight_store.extend([w_packed, scales])
        return w_packed, scales

    def _register(self, w: np.ndarray, s: np.ndarray) -> None:
        rc = self._lib.tl_register_weights(_np_ptr(w, ctypes.c_int8), _np_ptr(s), w.shape[0], w.shape[1])
        if rc != 0:
            _lin.check(self._lib, "tl_register_weights")

    def _register_layer(self, l_idx: int, layer: Mapping[str, np.ndarray]) -> None:
        q = {name: self._quantize_and_keep(layer[name]) for name in PROJECTIONS}
        # fused Q||K||V [4096 x 2048] and gate||up [12288 x 2048] (reference :290-302)
        qkv_w = np.ascontiguousarray(np.concatenate([q["q_proj"][0], q["k_proj"][0], q["v_proj"][0]], axis=0))
        qkv_s = np.ascontiguousarray(np.concatenate([q["q_proj"][1], q["k_proj"][1], q["v_proj"][1]]))
        gu_w = np.ascontiguousarray(np.concatenate([q["gate_proj"][0], q["up_proj"][0]], axis=0))
        gu_s = np.ascontiguousarray(np.concatenate([q["gate_proj"][1], q["up_proj"][1]]))
        self._weight_store.extend([qkv_w, qkv_s, gu_w, gu_s])
        entry = dict(q)
        entry["qkv_proj"] = (qkv_w, qkv_s)
        entry["gate_up_proj"] = (gu_w, gu_s)
        if all(n in layer for n in NORMS):
            norms = [np.ascontiguousarray(layer[n], dtype=np.float32) for n in NORMS]
            self._weight_store.extend(norms)
            self._set_device_layer(l_idx, entry, norms)
        for w, s in entry.values():
            self._register(w, s)
        self.layers.append(entry)

    # -- device layer loop (reference decoder.py:197-210, :304-317, :322-370) --
    def _init_device_loop(self) -> None:
        if self._c_model:
            return
        lib = self._lib
        max_seq = self._max_seq
        self._c_model = lib.decoder_model_alloc()
        self._c_cache = lib.decoder_cache_alloc(max_seq)
        self._c_scratch = lib.decoder_scratch_alloc_fn(max_seq)
        if not (self._c_model and self._c_cache and self._c_scratch):
            _lin.check(lib, "decoder handles")
            raise RuntimeError("decoder handle allocation failed")
        half = HEAD_DIM // 2
        self._cos_tab = np.empty((max_seq, half), dtype=np.float32)
        self._sin_tab = np.empty((max_seq, half), dtype=np.float32)
        lib.decoder_precompute_rope(_np_ptr(self._cos_tab), _np_ptr(self._sin_tab), max_seq, HEAD_DIM,
                                    (ctypes.c_int * 3)(*MROPE_SECTIONS), (ctypes.c_float * 3)(*MROPE_THETA_BASE))
        _lin.check(lib, "decoder_precompute_rope")

    def _set_device_layer(self, l_idx: int, q: Mapping[str, tuple], norms: List[np.ndarray]) -> None:
        """The layer's seven projections, four norms and the fused Q||K||V and
        gate||up, registered through decoder_set_layer_weights_v32 as the
        reference's _register_layer does (decoder.py:304-317)."""
        self._init_device_loop()
        args = []
        for name in PROJECTIONS + ("qkv_proj", "gate_up_proj"):
            w, s_ = q[name]
            args.append((_np_ptr(w, ctypes.c_int8), _np_ptr(s_)))
        flat = [p for pair in args[:len(PROJECTIONS)] for p in pair]
        flat += [_np_ptr(n) for n in norms]
        flat += [p for pair in args[len(PROJECTIONS):] for p in pair]
        self._lib.decoder_set_layer_weights_v32(self._c_model, l_idx, *flat)
        _lin.check(self._lib, "decoder_set_layer_weights_v32")

    def reset(self) -> None:
        """Clear the KV cache for a new sequence (reference :322-323)."""
        self._lib.decoder_cache_clear(self._c_cache)

    def set_rope_offset(self, offset: int) -> None:
        self._lib.decoder_cache_set_rope_offset(self._c_cache, offset)

    @property
    def cache_len(self) -> int:
        return self._lib.tl_decoder_cache_len(self._c_cache)

    def set_prefill_w8a8(self, on: bool) -> None:
        """Prefill linears on per-token int8 activations (W8A8) instead of the
        reference decoder's fp32 activations."""
        self._init_device_loop()
        if self._lib.tl_decoder_set_prefill_w8a8(self._c_model, 1 if on else 0) != 0:
            _lin.check(self._lib, "tl_decoder_set_prefill_w8a8")

    def prefill(self, hidden_np: np.ndarray, chunk: int = 0) -> np.ndarray:
        """Prefill hidden [seq_len, HIDDEN_DIM] at sequential positions
        (decoder_prefill_step; with chunk > 0 decoder_chunked_prefill_step,
        whose chunks attend to the whole cache)."""
        assert hidden_np.ndim == 2 and hidden_np.shape[1] == HIDDEN_DIM
        h = np.array(hidden_np, dtype=np.float32, copy=True)
        if chunk > 0:
            self._lib.decoder_chunked_prefill_step(self._c_model, self._c_cache, _np_ptr(h), self._c_scratch,
                                                   _np_ptr(self._cos_tab), _np_ptr(self._sin_tab), h.shape[0], chunk)
        else:
            self._lib.decoder_prefill_step(self._c_model, self._c_cache, _np_ptr(h), self._c_scratch,
                                           _np_ptr(self._cos_tab), _np_ptr(self._sin_tab), h.shape[0])
        _lin.check(self._lib, "decoder_prefill_step")
        return h

    def prefill_3d(self, hidden_np: np.ndarray, position_ids_3d: np.ndarray) -> np.ndarray:
        """Prefill with 3-D M-RoPE position ids [3, seq_len] (reference
        :325-358: decoder_build_rope_3d, then decoder_prefill_step_3d)."""
        assert hidden_np.ndim == 2 and hidden_np.shape[1] == HIDDEN_DIM
        h = np.ascontiguousarray(hidden_np, dtype=np.float32).copy()
        S = h.shape[0]
        pos = np.ascontiguousarray(position_ids_3d, dtype=np.int32)
        assert pos.shape == (3, S), f"position_ids_3d shape {pos.shape} != (3, {S})"
        half = HEAD_DIM // 2
        tc = np.empty((S, half), np.float32)
        ts = np.empty((S, half), np.float32)
        self._lib.decoder_build_rope_3d(_np_ptr(tc), _np_ptr(ts), pos.ctypes.data_as(ctypes.POINTER(ctypes.c_int)), S,
                                        HEAD_DIM, (ctypes.c_int * 3)(*MROPE_SECTIONS),
                                        (ctypes.c_float * 3)(*MROPE_THETA_BASE))
        self._lib.decoder_prefill_step_3d(self._c_model, self._c_cache, _np_ptr(h), self._c_scratch, _np_ptr(tc),
                                          _np_ptr(ts), S)
        _lin.check(self._lib, "decoder_prefill_step_3d")
        return h

    def step(self, hidden_np: np.ndarray) -> np.ndarray:
        """One decode step of every layer for hidden [1, HIDDEN_DIM]
        (reference :360-370, decoder_decode_step)."""
        assert hidden_np.ndim == 2 and hidden_np.shape == (1, HIDDEN_DIM)
        hidden_c = np.array(hidden_np, dtype=np.float32, copy=True)
        self._lib.decoder_decode_step(self._c_model, self._c_cache, _np_ptr(hidden_c), self._c_scratch,
                                      _np_ptr(self._cos_tab), _np_ptr(self._sin_tab))
        _lin.check(self._lib, "decoder_decode_step")
        return hidden_c

    def read_cache(self, layer: int):
        """(K, V) of one layer, each [8, max_seq, 128] fp32."""
        k = np.empty((NUM_KV_HEADS, self._max_seq, HEAD_DIM), np.float32)
        v = np.empty_like(k)
        if self._lib.tl_decoder_read_cache(self._c_cache, layer, _np_ptr(k), _np_ptr(v)) != 0:
            _lin.check(self._lib, "tl_decoder_read_cache")
        return k, v

    def generate_greedy(self, first_token: int, n_steps: int, embed_dev, lm_head_dev: "_lin.DeviceWeights"):
        """Greedy decode loop on the device (reference :494-507 with
        do_sample=False): n_steps tokens after first_token; embed_dev is a
        device tensor [vocab, HIDDEN_DIM] fp32, lm_head_dev the packed lm_head."""
        tokens = np.empty(n_steps, np.int32)
        fn = None if self._final_norm_w is None else _np_ptr(self._final_norm_w)
        rc = self._lib.tl_decoder_generate(self._c_model, self._c_cache, self._c_scratch, lm_head_dev.handle, fn,
                                           embed_dev.data_ptr(), int(first_token), int(n_steps),
                                           tokens.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                                           _np_ptr(self._cos_tab), _np_ptr(self._sin_tab))
        if rc != 0:
            _lin.check(self._lib, "tl_decoder_generate")
        return tokens

    def close(self) -> None:
        lib = self._lib
        for attr, fn in (("_c_model", lib.decoder_model_free), ("_c_cache", lib.decoder_cache_free),
                         ("_c_scratch", lib.decoder_scratch_free_fn)):
            h = getattr(self, attr, None)
            if h:
                fn(h)
                setattr(self, attr, None)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- core operations ------------------------------------------------------
    def project(self, l_idx: int, name: str, x: np.ndarray, out: Optional[np.ndarray] = None) -> np.ndarray:
        """y = w8a32_linear(x, W[name]) with the reference's call convention
        (bias NULL, scratch ignored): batch==1 rows take the int8 GEMV."""
        w, s = self.layers[l_idx][name]
        x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
        batch, K = x.shape
        M = w.shape[0]
        y = out if out is not None else np.empty((batch, M), np.float32)
        self._lib.w8a32_linear(_np_ptr(x), _np_ptr(w, ctypes.c_int8), _np_ptr(s), None, _np_ptr(y), None,
                               ctypes.c_int(batch), ctypes.c_int(M), ctypes.c_int(K))
        _lin.check(self._lib, "w8a32_linear")
        return y

    def get_logits(self, h_np: np.ndarray) -> np.ndarray:
        """Final RMSNorm of the last row (numpy, as reference :444-448), then the
        lm_head GEMV w8a32_linear(batch=1, N=vocab) (:449-459)."""
        if self._lm_head_w is None:
            raise RuntimeError("Decoder has no lm_head")
        h = np.atleast_2d(h_np)[-1]
        rms = np.sqrt(np.mean(h * h) + RMS_EPS)
        h_normed = (h / rms) * self._final_norm_w if self._final_norm_w is not None else h / rms
        x = np.ascontiguousarray(h_normed.reshape(1, self._lm_head_K), dtype=np.float32)
        self._lib.w8a32_linear(_np_ptr(x), _np_ptr(self._lm_head_w, ctypes.c_int8), _np_ptr(self._lm_head_s),
                               None, _np_ptr(self._logits_buf), _np_ptr(self._lm_head_scratch),
                               ctypes.c_int(1), ctypes.c_int(self._lm_head_M), ctypes.c_int(self._lm_head_K))
        _lin.check(self._lib, "w8a32_linear")
        return self._logits_buf

    def next_token(self, h_np: np.ndarray) -> int:
        """Greedy next token, get_logits + sample in one library call
        (tl_lm_head_argmax): the same final RMSNorm in numpy's float32 order,
        the same lm_head GEMV, the first index of the largest logit; only the
        4-byte token id comes back instead of the vocab-sized logits."""
        if self._lm_head_w is None:
            raise RuntimeError("Decoder has no lm_head")
        h = np.ascontiguousarray(np.atleast_2d(h_np)[-1], dtype=np.float32)
        return _lin.lm_head_argmax(h, self._final_norm_w, self._lm_head_w, self._lm_head_s)

    @staticmethod
    def sample(logits_1d: np.ndarray) -> int:
        """Greedy branch of _sample (reference :463-464): first index of the max."""
        return int(np.argmax(logits_1d))
