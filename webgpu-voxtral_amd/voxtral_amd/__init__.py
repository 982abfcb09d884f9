"""Python host binding of libvoxtral_amd.so (include/voxtral_engine.h).

`VoxtralEngine` mirrors the public surface of the reference class
(src/engine.ts:291-2633 of svenflow/webgpu-voxtral): same method names in
snake_case, same argument meaning, same error messages.  Every call goes
through the C ABI into the HIP engine; there is no CPU fallback -- importing
works without a GPU, but creating an engine needs the built library and a
HIP device, and fails loudly otherwise.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
# VOXTRAL_AMD_LIB selects another build of the library (e.g. the host-
# sanitizer build of `make asan`)
LIB_PATH = os.environ.get("VOXTRAL_AMD_LIB") or os.path.join(PKG, "lib", "libvoxtral_amd.so")
HEADER = os.path.join(os.path.dirname(PKG), "include", "voxtral_engine.h")

VX_OK, VX_E_INVALID, VX_E_STATE, VX_E_DEVICE, VX_E_RANGE, VX_E_NOMEM = 0, -1, -2, -3, -4, -5
EMBED_TOKEN, EMBED_AUDIO, EMBED_PRECOMPUTED, EMBED_CODES = 0, 1, 2, 3
SAMPLE_TOP_P, SAMPLE_GREEDY, SAMPLE_TOP_P_HOST = 0, 1, 2
KERNEL_QKV, KERNEL_ATTN, KERNEL_OPROJ, KERNEL_GATEUP, KERNEL_DOWN = range(5)
KERNEL_NAMES = ["qkv", "attn", "oproj", "gateup", "down"]
# flow-matching kernels, time_kernel indices 5.. (VX_KERNEL_FM_*)
FM_KERNEL_NAMES = ["fm_qkv", "fm_attn", "fm_o", "fm_gateup", "fm_down", "fm_step_in"]


class VoxtralError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(msg)
        self.code = code


class Config(ctypes.Structure):
    """vx_config == defaultConfig (src/types.ts:70-122), backbone + fm."""
    _fields_ = [
        ("dim", ctypes.c_int32), ("n_layers", ctypes.c_int32),
        ("head_dim", ctypes.c_int32), ("hidden_dim", ctypes.c_int32),
        ("n_heads", ctypes.c_int32), ("n_kv_heads", ctypes.c_int32),
        ("vocab_size", ctypes.c_int32), ("rope_theta", ctypes.c_float),
        ("norm_eps", ctypes.c_float), ("fm_layers", ctypes.c_int32),
        ("nfe", ctypes.c_int32), ("cfg_alpha", ctypes.c_float),
        ("n_acoustic_out", ctypes.c_int32), ("semantic_vocab", ctypes.c_int32),
        ("acoustic_levels", ctypes.c_int32), ("audio_vocab", ctypes.c_int32),
        ("kv_f16", ctypes.c_int32),  # KV cache element type: 0 f32 (reference), 1 f16
        ("codec", ctypes.c_int32),   # 1: the codec decoder is part of the engine (default)
    ]


class GenerateOptions(ctypes.Structure):
    _fields_ = [("sampling", ctypes.c_int32), ("top_p", ctypes.c_double),
                ("temperature", ctypes.c_double), ("seed", ctypes.c_uint64),
                ("ignore_eos", ctypes.c_int32)]


class GenerateStats(ctypes.Structure):
    _fields_ = [("backbone_ms", ctypes.c_double), ("fm_ms", ctypes.c_double),
                ("codec_ms", ctypes.c_double), ("total_ms", ctypes.c_double),
                ("frames_generated", ctypes.c_int32)]


FRAME_CB = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_int32, ctypes.c_uint32,
                            ctypes.POINTER(ctypes.c_uint32))
STAGE_CB = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_int32, ctypes.c_double)
_LOAD_CB = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_char_p,
                            ctypes.c_char_p, ctypes.c_uint64)

FRAME_SAMPLES = 1920  # 80 ms of 24 kHz audio per frame (VX_FRAME_SAMPLES)
NAC = 36
# debugCodecDecode's intermediates in decoder order (VX_CODEC_STOP_* 0..9)
CODEC_STOPS = ["concat", "after_input_conv",
               "after_stage0_transformer", "after_stage0_conv_up",
               "after_stage1_transformer", "after_stage1_conv_up",
               "after_stage2_transformer", "after_stage2_conv_up",
               "after_stage3_transformer", "audio"]

_VP = ctypes.c_void_p
_I32 = ctypes.c_int32
_SIGS = {
    "vx_config_default": (_I32, [ctypes.POINTER(Config)]),
    "vx_create": (_I32, [ctypes.POINTER(Config), _I32, ctypes.POINTER(_VP)]),
    "vx_destroy": (None, [_VP]),
    "vx_last_error": (ctypes.c_char_p, [_VP]),
    "vx_load_tensor": (_I32, [_VP, ctypes.c_char_p, _VP, ctypes.c_size_t, _VP, _I32]),
    "vx_init_synthetic": (_I32, [_VP, ctypes.c_uint64, ctypes.c_float]),
    "vx_read_tensor": (_I32, [_VP, ctypes.c_char_p, _VP, ctypes.c_size_t]),
    "vx_is_ready": (_I32, [_VP]),
    "vx_prefill": (_I32, [_VP, _VP, _I32, _I32, _I32, _VP]),
    "vx_load_safetensors": (_I32, [_VP, ctypes.c_char_p, _VP, _VP]),
    "vx_load_safetensors_progress": (_I32, [_VP, ctypes.c_char_p, _VP, _VP, _VP, _VP]),
    "vx_missing_tensor": (_I32, [_VP, ctypes.c_char_p, _I32]),
    "vx_bf16_to_f16": (None, [_VP, _VP, ctypes.c_size_t]),
    "vx_f32_to_f16_trunc": (None, [_VP, _VP, ctypes.c_size_t]),
    "vx_sample_top_p": (_I32, [_VP, _VP, _I32, _I32, ctypes.c_double, ctypes.c_double, _VP, _I32,
                               _VP]),
    "vx_sample_top_p_noalloc": (_I32, [_VP, _I32, _I32, ctypes.c_double, ctypes.c_double, _VP, _VP]),
    "vx_reset": (_I32, [_VP]),
    "vx_position": (_I32, [_VP]),
    "vx_set_position": (_I32, [_VP, _I32]),
    "vx_backbone_step": (_I32, [_VP, _I32, _I32, _VP, _I32, _VP, _VP]),
    "vx_backbone_step_layers": (_I32, [_VP, _I32, _I32, _VP, _VP]),
    "vx_debug_backbone_layers": (_I32, [_VP, _I32, _I32, _VP, _VP, _VP]),
    "vx_fm_forward": (_I32, [_VP, _VP, _VP, _VP, _VP]),
    "vx_set_semantic_code": (_I32, [_VP, ctypes.c_uint32]),
    "vx_set_acoustic_codes": (_I32, [_VP, _VP]),
    "vx_get_codes": (_I32, [_VP, _VP, _VP]),
    "vx_read": (_I32, [_VP, ctypes.c_char_p, _VP, ctypes.c_size_t]),
    "vx_write": (_I32, [_VP, ctypes.c_char_p, _VP, ctypes.c_size_t]),
    "vx_write_kv": (_I32, [_VP, _I32, _I32, _I32, _I32, _VP]),
    "vx_read_kv": (_I32, [_VP, _I32, _I32, _I32, _I32, _VP]),
    "vx_fill_kv_synthetic": (_I32, [_VP, ctypes.c_uint64, _I32]),
    "vx_generate_options_default": (None, [ctypes.POINTER(GenerateOptions)]),
    "vx_generate": (_I32, [_VP, _VP, _I32, _I32, _I32, _VP, _I32, ctypes.POINTER(GenerateOptions),
                           FRAME_CB, STAGE_CB, _VP, _VP, _VP, _VP, ctypes.POINTER(GenerateStats)]),
    "vx_codec_decode": (_I32, [_VP, _VP, _VP, _I32, _VP]),
    "vx_codec_decode_debug": (_I32, [_VP, _VP, _VP, _I32, _I32, _VP, ctypes.c_size_t]),
    "vx_codec_stop_count": (ctypes.c_size_t, [_I32, _I32]),
    "vx_tokenizer_create": (_I32, [_VP, _VP, _VP, _I32, _I32, ctypes.POINTER(_VP)]),
    "vx_tokenizer_destroy": (None, [_VP]),
    "vx_tokenizer_encode_pieces": (_I32, [_VP, _VP, _VP, _I32, _VP, ctypes.c_int64,
                                          ctypes.POINTER(ctypes.c_int64)]),
    "vx_time_backbone_steps": (_I32, [_VP, _I32, _I32, ctypes.POINTER(ctypes.c_float)]),
    "vx_time_frames": (_I32, [_VP, _I32, ctypes.POINTER(ctypes.c_float)]),
    "vx_time_kernel": (_I32, [_VP, _I32, _I32, ctypes.POINTER(ctypes.c_float),
                              ctypes.POINTER(ctypes.c_double)]),
    "vx_debug_timeline": (_I32, [_VP, _I32, _VP, _I32, ctypes.POINTER(_I32)]),
    "vx_synchronize": (_I32, [_VP]),
}

_lib = None


def load_library(path=None):
    """Loads libvoxtral_amd.so; raises if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    path = path or LIB_PATH
    if not os.path.exists(path):
        raise RuntimeError(f"libvoxtral_amd.so not built ({path}); run __graft_entry__.build()")
    lib = ctypes.CDLL(path)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def exported_symbols():
    return list(_SIGS)


def bf16_to_f16(bits):
    """convertBF16toF16 (src/weights.ts:94-138) on uint16 BF16 bits."""
    a = np.ascontiguousarray(bits, np.uint16)
    out = np.empty_like(a)
    load_library().vx_bf16_to_f16(a.ctypes.data, out.ctypes.data, a.size)
    return out


def f32_to_f16_trunc(values):
    """float32ToFloat16 (src/weights.ts:222-232): truncating, no subnormals."""
    a = np.ascontiguousarray(values, np.float32)
    out = np.empty(a.shape, np.uint16)
    load_library().vx_f32_to_f16_trunc(a.ctypes.data, out.ctypes.data, a.size)
    return out


def sample_top_p_noalloc(logits, valid, top_p, temperature, state):
    """The device top-p of VoxtralEngine.sample_top_p without an engine or
    any allocation (vx_sample_top_p_noalloc: the library's own staging array,
    at most 9216 logits); returns (code, next splitmix64 state)."""
    L = load_library()
    lg = np.ascontiguousarray(logits, np.float32)
    st = ctypes.c_uint64(state)
    code = ctypes.c_uint32()
    rc = L.vx_sample_top_p_noalloc(lg.ctypes.data, lg.size, int(valid), float(top_p),
                                   float(temperature), ctypes.byref(st), ctypes.byref(code))
    if rc != VX_OK:
        raise VoxtralError(rc, L.vx_last_error(None).decode())
    return code.value, st.value


def default_config(**over):
    c = Config()
    load_library().vx_config_default(ctypes.byref(c))
    for k, v in over.items():
        setattr(c, k, v)
    return c


def _ptr(a):
    return a.ctypes.data if a is not None else None


def _f32(a, n=None):
    a = np.ascontiguousarray(a, np.float32)
    if n is not None and a.size != n:
        raise ValueError(f"expected {n} float32 values, got {a.size}")
    return a


class VoxtralEngine:
    """MI355X engine with the reference VoxtralEngine surface."""

    def __init__(self, config=None, max_seq_len=4096):
        self._lib = load_library()
        self.config = config if config is not None else default_config()
        self.max_seq_len = int(max_seq_len)
        self._h = None

    # -- lifecycle (constructor :301-304, init :313-340, destroy :2621) --
    def init(self):
        h = ctypes.c_void_p()
        rc = self._lib.vx_create(ctypes.byref(self.config), self.max_seq_len, ctypes.byref(h))
        if rc != VX_OK:
            raise VoxtralError(rc, self._lib.vx_last_error(None).decode())
        self._h = h
        return self

    def destroy(self):
        if self._h:
            self._lib.vx_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.destroy()

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass

    def _check(self, rc):
        if rc != VX_OK:
            raise VoxtralError(rc, self._lib.vx_last_error(self._h).decode())

    # -- weights (loadWeights :539, organizeWeights :659-743) --
    def load_tensor(self, name, f16_bits, shape=None):
        a = np.ascontiguousarray(f16_bits)
        if a.dtype == np.float16:
            a = a.view(np.uint16)
        if a.dtype != np.uint16:
            raise TypeError("weights are float16 (or their uint16 bit patterns)")
        shape = tuple(shape) if shape is not None else a.shape
        sh = (ctypes.c_int64 * len(shape))(*shape)
        self._check(self._lib.vx_load_tensor(self._h, name.encode(), a.ctypes.data, a.size,
                                             ctypes.cast(sh, ctypes.c_void_p), len(shape)))

    def load_weights(self, tensors):
        """tensors: mapping of reference tensor name -> float16 array."""
        for name, arr in tensors.items():
            self.load_tensor(name, arr)

    def read_tensor(self, name, numel):
        out = np.empty(int(numel), np.uint16)
        self._check(self._lib.vx_read_tensor(self._h, name.encode(), out.ctypes.data, out.size))
        return out

    def load_safetensors(self, path, on_progress=None):
        """loadWeightsFromHF from a local safetensors file; returns
        (tensors loaded, tensors skipped).  on_progress(dict) after each
        tensor, with HFLoadProgress's fields (src/weights.ts:465-472):
        loaded, total, component, tensor, cached (False), bytesDownloaded
        (bytes read from the file)."""
        n, k = ctypes.c_int32(), ctypes.c_int32()
        if on_progress is None:
            self._check(self._lib.vx_load_safetensors(self._h, os.fsencode(path), ctypes.byref(n),
                                                      ctypes.byref(k)))
            return n.value, k.value
        errors = []

        def cb(_user, loaded, total, component, tensor, nbytes):
            if errors:
                return
            try:
                on_progress({"loaded": loaded, "total": total, "component": component.decode(),
                             "tensor": tensor.decode(), "cached": False, "bytesDownloaded": nbytes})
            except BaseException as e:  # re-raised after the load returns
                errors.append(e)
        c_cb = _LOAD_CB(cb)
        rc = self._lib.vx_load_safetensors_progress(self._h, os.fsencode(path), c_cb, None,
                                                    ctypes.byref(n), ctypes.byref(k))
        if errors:
            raise errors[0]
        self._check(rc)
        return n.value, k.value

    def missing_tensor(self):
        """The first weight not loaded yet (organizeWeights' "Missing weight",
        src/engine.ts:663-667), or None."""
        buf = ctypes.create_string_buffer(512)
        return buf.value.decode() if self._lib.vx_missing_tensor(self._h, buf, len(buf)) else None

    def init_synthetic(self, seed=0, std=0.02):
        self._check(self._lib.vx_init_synthetic(self._h, seed, std))

    @property
    def is_ready(self):
        return bool(self._h) and bool(self._lib.vx_is_ready(self._h))

    # -- state --
    def reset(self):
        self._check(self._lib.vx_reset(self._h))

    @property
    def position(self):
        return self._lib.vx_position(self._h)

    @position.setter
    def position(self, p):
        self._check(self._lib.vx_set_position(self._h, int(p)))

    def write_kv(self, layer, which, pos0, rows):
        """rows: [npos, n_kv_heads*head_dim] values (f32; an f16 cache rounds)."""
        a = np.ascontiguousarray(rows, np.float32)
        kvd = self.config.n_kv_heads * self.config.head_dim
        npos = a.size // kvd
        self._check(self._lib.vx_write_kv(self._h, layer, which, pos0, npos, a.ctypes.data))

    def read_kv(self, layer, which, pos0, npos):
        kvd = self.config.n_kv_heads * self.config.head_dim
        out = np.empty((npos, kvd), np.float32)
        self._check(self._lib.vx_read_kv(self._h, layer, which, pos0, npos, out.ctypes.data))
        return out

    def fill_kv_synthetic(self, seed, npos):
        self._check(self._lib.vx_fill_kv_synthetic(self._h, seed, npos))

    # -- backbone (backboneStep :814-1042) --
    def backbone_step(self, token=0, mode=EMBED_TOKEN, precomputed=None, lm_head=False,
                      read_normed=True):
        pre = None
        if precomputed is not None:
            pre = _f32(precomputed, self.config.dim)
            mode = EMBED_PRECOMPUTED
        am = np.zeros(1, np.uint32)
        normed = np.empty(self.config.dim, np.float32) if read_normed else None
        self._check(self._lib.vx_backbone_step(self._h, int(token), int(mode), _ptr(pre),
                                               int(bool(lm_head)), _ptr(am), _ptr(normed)))
        return (int(am[0]) if lm_head else None), normed

    def prefill(self, tokens, audio_token_start=0, audio_token_count=0, voice_embeddings=None):
        """The prefill loop of generate() (src/engine.ts:2457-2472) as batched
        GEMMs: KV cache, residual stream, W.normed and position as after one
        step per token (no LM head)."""
        toks = np.ascontiguousarray(tokens, np.int32)
        voice = None
        if voice_embeddings is not None and audio_token_count > 0:
            voice = _f32(voice_embeddings)
            if voice.size < audio_token_count * self.config.dim:
                raise ValueError("voiceEmbeddings shorter than audioTokenCount rows")
        self._check(self._lib.vx_prefill(self._h, toks.ctypes.data, toks.size, audio_token_start,
                                         audio_token_count if voice is not None else 0,
                                         _ptr(voice)))

    def backbone_step_and_read(self, token_id, use_audio_embedding=False):
        """backboneStepAndRead (:2333-2342): next-token argmax."""
        am, _ = self.backbone_step(token_id, EMBED_AUDIO if use_audio_embedding else EMBED_TOKEN,
                                   lm_head=True, read_normed=False)
        return am

    def debug_backbone_step_full(self, token_id, use_audio_embedding=False):
        """debugBackboneStepFull (:2348-2357): final-norm hidden state."""
        return self.backbone_step(token_id, EMBED_AUDIO if use_audio_embedding else EMBED_TOKEN)[1]

    def debug_backbone_layer_by_layer(self, token_id, precomputed=None, use_audio_embedding=False):
        """debugBackboneLayerByLayer (:2106-2287): the embedding, per layer
        attn_norm, attn_out (hidden after the attention residual), ffn_norm
        and ffn_out (hidden after the FFN residual), the final norm and the
        last hidden state."""
        c = self.config
        emb = np.empty(c.dim, np.float32)
        out = np.empty((c.n_layers, 4, c.dim), np.float32)
        pre = _f32(precomputed, c.dim) if precomputed is not None else None
        mode = EMBED_PRECOMPUTED if pre is not None else (EMBED_AUDIO if use_audio_embedding else EMBED_TOKEN)
        self._check(self._lib.vx_debug_backbone_layers(self._h, int(token_id), mode, _ptr(pre),
                                                       emb.ctypes.data, out.ctypes.data))
        names = ("attn_norm", "attn_out", "ffn_norm", "ffn_out")
        return {"embed": emb,
                "layers": [{n: out[i, k] for k, n in enumerate(names)} for i in range(c.n_layers)],
                "final_norm": self.debug_read("normed", c.dim), "hidden": out[-1, 3].copy()}

    def backbone_step_layers(self, token_id, mode=EMBED_TOKEN, precomputed=None):
        """Hidden state after each attention and each FFN residual,
        [n_layers][2][dim] (vx_backbone_step_layers)."""
        c = self.config
        out = np.empty((c.n_layers, 2, c.dim), np.float32)
        pre = _f32(precomputed, c.dim) if precomputed is not None else None
        if pre is not None:
            mode = EMBED_PRECOMPUTED
        self._check(self._lib.vx_backbone_step_layers(self._h, int(token_id), mode, _ptr(pre),
                                                      out.ctypes.data))
        return out

    # -- FM (fmForward :1240-1380) --
    def debug_fm_step(self, debug_noise=None):
        """debugFMStep (:2363-2380)."""
        noise = _f32(debug_noise, 36) if debug_noise is not None else None
        sem = np.empty(self.config.semantic_vocab, np.float32)
        codes = np.empty(36, np.uint32)
        xf = np.empty(36, np.float32)
        self._check(self._lib.vx_fm_forward(self._h, _ptr(noise), sem.ctypes.data,
                                            codes.ctypes.data, xf.ctypes.data))
        return {"semantic_logits": sem, "acoustic_codes": codes, "x_final": xf}

    def fm_step_and_read(self):
        """fmStepAndRead (:2386-2396): acoustic codes of one frame."""
        codes = np.empty(36, np.uint32)
        self._check(self._lib.vx_fm_forward(self._h, None, None, codes.ctypes.data, None))
        return codes

    def set_semantic_code(self, code):
        self._check(self._lib.vx_set_semantic_code(self._h, int(code)))

    def set_acoustic_codes(self, codes):
        c = np.ascontiguousarray(codes, np.uint32)
        self._check(self._lib.vx_set_acoustic_codes(self._h, c.ctypes.data))

    def get_codes(self):
        s = np.zeros(1, np.uint32)
        c = np.zeros(36, np.uint32)
        self._check(self._lib.vx_get_codes(self._h, s.ctypes.data, c.ctypes.data))
        return int(s[0]), c

    def debug_read(self, buffer_name, count=16):
        """debugRead (:2062-2067)."""
        out = np.empty(int(count), np.float32)
        self._check(self._lib.vx_read(self._h, buffer_name.encode(), out.ctypes.data, out.size))
        return out

    def debug_write(self, buffer_name, values):
        """queue.writeBuffer into `normed` or `hidden` (teacher forcing)."""
        v = _f32(values)
        self._check(self._lib.vx_write(self._h, buffer_name.encode(), v.ctypes.data, v.size))

    # -- generate (:2416-2616) --
    def generate(self, tokens, audio_token_start, audio_token_count, voice_embeddings,
                 max_frames=500, on_frame=None, on_stage=None, sampling="top_p", seed=0,
                 top_p=0.9, temperature=0.8, ignore_eos=False):
        toks = np.ascontiguousarray(tokens, np.int32)
        voice = None
        if voice_embeddings is not None and audio_token_count > 0:
            voice = _f32(voice_embeddings)
            if voice.size < audio_token_count * self.config.dim:
                raise ValueError("voiceEmbeddings shorter than audioTokenCount rows")
        opt = GenerateOptions()
        self._lib.vx_generate_options_default(ctypes.byref(opt))
        opt.sampling = {"greedy": SAMPLE_GREEDY, "top_p": SAMPLE_TOP_P,
                        "top_p_host": SAMPLE_TOP_P_HOST}[sampling]
        opt.top_p, opt.temperature, opt.seed, opt.ignore_eos = top_p, temperature, seed, int(ignore_eos)
        sem = np.zeros(max(1, max_frames), np.uint32)
        ac = np.zeros((max(1, max_frames), 36), np.uint32)
        audio = np.zeros(max(1, max_frames) * FRAME_SAMPLES, np.float32) if self.config.codec else None
        stages = ["backbone", "fm", "codec"]

        def _frame(user, f, s, codes):
            if on_frame:
                on_frame(f, s, np.ctypeslib.as_array(codes, (36,)).copy())

        def _stage(user, st, done):
            if on_stage:
                on_stage(stages[st], None if done < 0 else done)

        fcb, scb = FRAME_CB(_frame), STAGE_CB(_stage)
        stats = GenerateStats()
        self._check(self._lib.vx_generate(self._h, toks.ctypes.data, toks.size, audio_token_start,
                                          audio_token_count, _ptr(voice), max_frames,
                                          ctypes.byref(opt), fcb, scb, None, sem.ctypes.data,
                                          ac.ctypes.data, _ptr(audio), ctypes.byref(stats)))
        n = stats.frames_generated
        return {
            "semanticCodes": [int(v) for v in sem[:n]],
            "acousticCodes": [list(map(int, r)) for r in ac[:n]],
            # codecDecode of the frames (empty for an engine without the codec)
            "audio": audio[:n * FRAME_SAMPLES].copy() if audio is not None else np.zeros(0, np.float32),
            "stats": {"backboneMs": stats.backbone_ms, "fmMs": stats.fm_ms,
                      "codecMs": stats.codec_ms, "totalMs": stats.total_ms,
                      "framesGenerated": n},
        }

    # -- codec decoder (:1402-1985) --
    def _codes(self, semantic, acoustic):
        sem = np.ascontiguousarray(semantic, np.uint32).ravel()
        ac = np.ascontiguousarray(acoustic, np.uint32).ravel()
        if ac.size != NAC * sem.size:
            raise ValueError("acousticCodes must hold 36 codes per frame")
        return sem, ac

    def codec_decode(self, semantic_codes, acoustic_codes):
        """codecDecode (:1402-1713): codes [T], [T][36] -> 24 kHz samples [T * 1920]."""
        sem, ac = self._codes(semantic_codes, acoustic_codes)
        out = np.empty(max(1, sem.size * FRAME_SAMPLES), np.float32)
        self._check(self._lib.vx_codec_decode(self._h, sem.ctypes.data, ac.ctypes.data, sem.size,
                                              out.ctypes.data))
        return out[:sem.size * FRAME_SAMPLES]

    def codec_decode_to(self, semantic_codes, acoustic_codes, stop):
        """The decoder up to one intermediate of debugCodecDecode (CODEC_STOPS)."""
        sem, ac = self._codes(semantic_codes, acoustic_codes)
        k = CODEC_STOPS.index(stop)
        n = self._lib.vx_codec_stop_count(sem.size, k)
        out = np.empty(max(1, n), np.float32)
        self._check(self._lib.vx_codec_decode_debug(self._h, sem.ctypes.data, ac.ctypes.data,
                                                    sem.size, k, out.ctypes.data, out.size))
        return out[:n]

    def debug_codec_decode(self, semantic_codes, acoustic_codes):
        """debugCodecDecode (:1719-1985): every intermediate by name."""
        out = {name: self.codec_decode_to(semantic_codes, acoustic_codes, name) for name in CODEC_STOPS}
        out["after_output_conv"] = out["audio"]
        return out

    def sample_top_p(self, logits, valid, top_p, temperature, state, on_device=True):
        """sampleTopP (src/engine.ts:247-289) on caller logits with indices 0
        and >= valid masked; returns (code, next splitmix64 state)."""
        lg = _f32(logits)
        st = ctypes.c_uint64(state)
        code = ctypes.c_uint32()
        self._check(self._lib.vx_sample_top_p(self._h, lg.ctypes.data, lg.size, int(valid),
                                               float(top_p), float(temperature), ctypes.byref(st),
                                               int(bool(on_device)), ctypes.byref(code)))
        return code.value, st.value

    # -- measurement (no reference counterpart) --
    def time_backbone_steps(self, n, hold_position=False, feedback=False):
        """n decode steps on the device; returns the event time in ms.
        hold_position: every step at the current position; feedback: each
        step's input is the previous step's W.normed (precomputed-embedding
        path), positions advancing."""
        if hold_position and feedback:
            raise ValueError("hold_position and feedback exclude each other")
        mode = 1 if hold_position else 2 if feedback else 0
        ms = ctypes.c_float()
        self._check(self._lib.vx_time_backbone_steps(self._h, int(n), mode, ctypes.byref(ms)))
        return ms.value

    def time_frames(self, n):
        ms = ctypes.c_float()
        self._check(self._lib.vx_time_frames(self._h, int(n), ctypes.byref(ms)))
        return ms.value

    def time_kernel(self, kernel, iters):
        us, b = ctypes.c_float(), ctypes.c_double()
        self._check(self._lib.vx_time_kernel(self._h, int(kernel), int(iters), ctypes.byref(us),
                                             ctypes.byref(b)))
        return us.value, b.value

    def timeline(self, reps=2):
        """Launch timeline of one held decode step (vx_debug_timeline): an
        [n][2] array of (earliest block start, latest block end) per launch on
        the GPU's 100 MHz wall clock, launch 6 l + k of layer l (k: QKV,
        attention partials, combine, O, gate/up, down), then the final norm."""
        n = 6 * self.config.n_layers + 1
        out = np.zeros(2 * n, np.uint64)
        got = ctypes.c_int32()
        self._check(self._lib.vx_debug_timeline(self._h, int(reps), out.ctypes.data, out.size,
                                                ctypes.byref(got)))
        return out.reshape(got.value, 2)

    def synchronize(self):
        self._check(self._lib.vx_synchronize(self._h))
