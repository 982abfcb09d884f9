"""ctypes binding of the CPU oracle (oracle/vx_oracle.c).

TEST INFRASTRUCTURE ONLY: the parity checker and the CPU baseline.  Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this.
The product never does.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "libvx_oracle.so")


def build(force=False):
    """Compile the oracle with its Makefile (gcc)."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


class Config(ctypes.Structure):
    _fields_ = [
        ("dim", ctypes.c_int), ("n_layers", ctypes.c_int),
        ("head_dim", ctypes.c_int), ("hidden_dim", ctypes.c_int),
        ("n_heads", ctypes.c_int), ("n_kv_heads", ctypes.c_int),
        ("vocab_size", ctypes.c_int), ("rope_theta", ctypes.c_float),
        ("norm_eps", ctypes.c_float), ("fm_layers", ctypes.c_int),
        ("nfe", ctypes.c_int), ("cfg_alpha", ctypes.c_float),
        ("n_acoustic_out", ctypes.c_int), ("semantic_vocab", ctypes.c_int),
        ("acoustic_levels", ctypes.c_int), ("audio_vocab", ctypes.c_int),
    ]


_lib = None
P = np.ctypeslib.ndpointer
F32 = P(dtype=np.float32, flags="C_CONTIGUOUS")
U16 = P(dtype=np.uint16, flags="C_CONTIGUOUS")
U32 = P(dtype=np.uint32, flags="C_CONTIGUOUS")
c_int, c_float, c_u64, c_size = ctypes.c_int, ctypes.c_float, ctypes.c_uint64, ctypes.c_size_t
c_vp = ctypes.c_void_p


def lib():
    global _lib
    if _lib is None:
        build()
        L = ctypes.CDLL(LIB_PATH)
        sig = {
            "vxo_default_config": (None, [ctypes.POINTER(Config)]),
            "vxo_f32_to_f16": (ctypes.c_uint16, [c_float]),
            "vxo_f16_to_f32": (c_float, [ctypes.c_uint16]),
            "vxo_splitmix64_next": (c_u64, [ctypes.POINTER(c_u64)]),
            "vxo_name_stream": (c_u64, [ctypes.c_char_p]),
            "vxo_normal": (c_float, [c_u64, c_u64, c_u64]),
            "vxo_gauss": (c_float, [c_u64, c_u64, c_u64]),
            "vxo_gen_gauss_f32": (None, [c_u64, c_u64, c_size, F32]),
            "vxo_gen_f32": (None, [c_u64, c_u64, c_size, c_float, c_float, F32]),
            "vxo_gen_f16": (None, [c_u64, c_u64, c_size, c_float, c_float, U16]),
            "vxo_matvec_f16": (None, [U16, F32, F32, c_int, c_int]),
            "vxo_rmsnorm": (None, [F32, U16, F32, c_int, c_float]),
            "vxo_embedding": (None, [U16, c_int, c_int, F32]),
            "vxo_rope": (None, [F32, c_int, c_int, c_int, c_float]),
            "vxo_attn_scores": (None, [F32, F32, F32, c_int, c_int, c_int, c_int]),
            "vxo_softmax": (None, [F32, c_int, c_int]),
            "vxo_attn_value": (None, [F32, F32, F32, c_int, c_int, c_int, c_int]),
            "vxo_swiglu": (None, [F32, F32, c_int]),
            "vxo_time_embedding": (None, [F32, c_int, c_float]),
            "vxo_cfg_combine": (None, [F32, F32, c_int, c_float]),
            "vxo_euler_step": (None, [F32, F32, c_int, c_float]),
            "vxo_fsq_quantize": (None, [F32, U32, c_int, c_int, c_int]),
            "vxo_argmax": (ctypes.c_uint32, [F32, c_int]),
            "vxo_multi_codebook_embed": (None, [U16, ctypes.c_uint32, U32, c_int, F32]),
            "vxo_bi_attention": (None, [F32, F32, F32, F32, F32, c_int, c_int, c_int, c_int]),
            "vxo_create": (c_vp, [ctypes.POINTER(Config), c_int]),
            "vxo_destroy": (None, [c_vp]),
            "vxo_set_weight": (c_int, [c_vp, ctypes.c_char_p, U16]),
            "vxo_init_synthetic": (c_int, [c_vp, c_u64, c_float]),
            "vxo_weight_numel": (c_size, [c_vp, ctypes.c_char_p]),
            "vxo_weight": (c_vp, [c_vp, ctypes.c_char_p]),
            "vxo_is_ready": (c_int, [c_vp]),
            "vxo_reset": (None, [c_vp]),
            "vxo_set_kv_f16": (None, [c_vp, c_int]),
            "vxo_position": (c_int, [c_vp]),
            "vxo_set_position": (None, [c_vp, c_int]),
            "vxo_buffer": (c_vp, [c_vp, ctypes.c_char_p, ctypes.POINTER(c_int)]),
            "vxo_kv": (c_vp, [c_vp, c_int, c_int]),
            "vxo_acoustic_codes": (c_vp, [c_vp]),
            "vxo_semantic_argmax": (ctypes.c_uint32, [c_vp]),
            "vxo_set_semantic_code": (None, [c_vp, ctypes.c_uint32]),
            "vxo_set_acoustic_codes": (None, [c_vp, U32]),
            "vxo_argmax_result": (ctypes.c_uint32, [c_vp]),
            "vxo_backbone_step": (None, [c_vp, c_int, c_int, c_vp, c_int]),
            "vxo_backbone_step_ex": (None, [c_vp, c_int, c_int, c_vp, c_int, c_vp]),
            "vxo_backbone_step_debug": (None, [c_vp, c_int, c_int, c_vp, c_vp, c_vp]),
            "vxo_backbone_step_codes": (None, [c_vp]),
            "vxo_fm_forward": (None, [c_vp, F32]),
            "vxo_fm_forward_batched": (None, [c_vp, F32]),
            "vxo_generate": (c_int, [c_vp, c_vp, c_int, c_int, c_int, c_vp, c_int, c_u64, c_int,
                                     c_vp, c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_vp]),
            # codec decoder (vx_oracle_codec.c)
            "vxo_normalize_codebook": (None, [U16, U16, U16, c_int, c_int, c_float]),
            "vxo_vq_lookup": (None, [U32, U16, F32, c_int, c_int, c_int]),
            "vxo_fsq_dequant": (None, [U32, F32, c_int, c_int, c_int]),
            "vxo_causal_conv1d": (None, [F32, U16, U16, F32, c_int, c_int, c_int, c_int, c_int]),
            "vxo_conv_transpose_scale": (None, [U16, U16, F32, c_int, c_int, c_int]),
            "vxo_conv_transpose1d": (None, [F32, U16, F32, F32, c_int, c_int, c_int, c_int, c_int]),
            "vxo_batched_rmsnorm": (None, [F32, U16, F32, c_int, c_int, c_float]),
            "vxo_batched_matvec_f16": (None, [U16, F32, F32, c_int, c_int, c_int]),
            "vxo_qk_norm": (None, [F32, U16, c_int, c_int, c_int, c_float]),
            "vxo_codec_attention": (None, [F32, F32, F32, F32, c_int, c_int, c_int, c_int]),
            "vxo_codec_create": (c_vp, []),
            "vxo_codec_destroy": (None, [c_vp]),
            "vxo_codec_n_weights": (c_int, [c_vp]),
            "vxo_codec_weight_name": (ctypes.c_char_p, [c_vp, c_int]),
            "vxo_codec_weight_numel": (c_size, [c_vp, ctypes.c_char_p]),
            "vxo_codec_weight": (c_vp, [c_vp, ctypes.c_char_p]),
            "vxo_codec_set_weight": (c_int, [c_vp, ctypes.c_char_p, U16]),
            "vxo_codec_init_synthetic": (c_int, [c_vp, c_u64, c_float]),
            "vxo_codec_stop_count": (c_size, [c_int, c_int]),
            "vxo_codec_decode": (c_int, [c_vp, U32, U32, c_int, c_int, F32]),
            "vxo_codec_decode_all": (c_int, [c_vp, U32, U32, c_int, c_vp]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def default_config(**over):
    c = Config()
    lib().vxo_default_config(ctypes.byref(c))
    for k, v in over.items():
        setattr(c, k, v)
    return c


# ---------------------------------------------------------------- numbers
def name_stream(name):
    return lib().vxo_name_stream(name.encode())


def gen_gauss_f32(seed, name, n):
    """n Box-Muller Gaussians of (seed, stream(name)): the FM noise generator."""
    out = np.empty(n, np.float32)
    lib().vxo_gen_gauss_f32(seed, name_stream(name), n, out)
    return out


def gen_f32(seed, name, n, mean=0.0, std=1.0):
    out = np.empty(n, np.float32)
    lib().vxo_gen_f32(seed, name_stream(name), n, mean, std, out)
    return out


def gen_f16(seed, name, n, mean=0.0, std=1.0):
    out = np.empty(n, np.uint16)
    lib().vxo_gen_f16(seed, name_stream(name), n, mean, std, out)
    return out


def f16_bits_to_f32(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


# ---------------------------------------------------------------- kernels
def matvec_f16(A_bits, x):
    M, K = A_bits.shape
    y = np.empty(M, np.float32)
    lib().vxo_matvec_f16(np.ascontiguousarray(A_bits), np.ascontiguousarray(x, np.float32), y, M, K)
    return y


def rmsnorm(x, w_bits, eps=1e-5):
    y = np.empty_like(x, dtype=np.float32)
    lib().vxo_rmsnorm(np.ascontiguousarray(x, np.float32), np.ascontiguousarray(w_bits), y, x.size, eps)
    return y


def rope(qk, head_dim, pos, theta):
    out = np.ascontiguousarray(qk, np.float32).copy()
    lib().vxo_rope(out, head_dim, pos, out.size // head_dim, theta)
    return out


def attention_decode(q, kcache, vcache, n_heads, n_kv_heads, head_dim, seq_len):
    """attnScore + softmax + attnValue; caches are [seq][n_kv*hd] f32."""
    scores = np.empty(n_heads * seq_len, np.float32)
    out = np.empty(n_heads * head_dim, np.float32)
    L = lib()
    kc = np.ascontiguousarray(kcache, np.float32)
    vc = np.ascontiguousarray(vcache, np.float32)
    L.vxo_attn_scores(np.ascontiguousarray(q, np.float32), kc, scores, n_heads, n_kv_heads, head_dim, seq_len)
    L.vxo_softmax(scores, n_heads, seq_len)
    L.vxo_attn_value(scores, vc, out, n_heads, n_kv_heads, head_dim, seq_len)
    return out, scores


def swiglu(g, u):
    out = np.ascontiguousarray(g, np.float32).copy()
    lib().vxo_swiglu(out, np.ascontiguousarray(u, np.float32), out.size)
    return out


def time_embedding(dim, t):
    out = np.empty(dim, np.float32)
    lib().vxo_time_embedding(out, dim, t)
    return out


def cfg_combine(vc, vu, alpha):
    out = np.ascontiguousarray(vc, np.float32).copy()
    lib().vxo_cfg_combine(out, np.ascontiguousarray(vu, np.float32), out.size, alpha)
    return out


def euler_step(x, v, dt):
    out = np.ascontiguousarray(x, np.float32).copy()
    lib().vxo_euler_step(out, np.ascontiguousarray(v, np.float32), out.size, dt)
    return out


def fsq_quantize(x, levels=21, offset=2):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.size, np.uint32)
    lib().vxo_fsq_quantize(x, out, x.size, levels, offset)
    return out


def argmax(x):
    return int(lib().vxo_argmax(np.ascontiguousarray(x, np.float32), x.size))


def multi_codebook_embed(table_bits, semantic_code, acoustic_codes, dim):
    out = np.empty(dim, np.float32)
    lib().vxo_multi_codebook_embed(np.ascontiguousarray(table_bits), semantic_code,
                                   np.ascontiguousarray(acoustic_codes, np.uint32), dim, out)
    return out


def bi_attention(q, k, v, n_heads, n_kv_heads, head_dim, seq_len=3):
    scores = np.empty(n_heads * seq_len * seq_len, np.float32)
    out = np.empty(seq_len * n_heads * head_dim, np.float32)
    lib().vxo_bi_attention(np.ascontiguousarray(q, np.float32), np.ascontiguousarray(k, np.float32),
                           np.ascontiguousarray(v, np.float32), scores, out,
                           n_heads, n_kv_heads, head_dim, seq_len)
    return out, scores


# ---------------------------------------------------------------- engine
class OracleEngine:
    """CPU restatement of VoxtralEngine's device state (src/engine.ts)."""

    def __init__(self, cfg=None, max_seq=4096):
        self.cfg = cfg if cfg is not None else default_config()
        self.max_seq = max_seq
        self._h = lib().vxo_create(ctypes.byref(self.cfg), max_seq)
        self._keep = {}

    def close(self):
        if self._h:
            lib().vxo_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def init_synthetic(self, seed=0, std=0.02):
        if lib().vxo_init_synthetic(self._h, seed, std) != 0:
            raise MemoryError("oracle synthetic weights")

    def set_weight(self, name, bits):
        bits = np.ascontiguousarray(bits, np.uint16).ravel()
        if bits.size != lib().vxo_weight_numel(self._h, name.encode()):
            raise ValueError(f"bad size for {name}")
        self._keep[name] = bits
        if lib().vxo_set_weight(self._h, name.encode(), bits) != 0:
            raise KeyError(name)

    def weight(self, name):
        n = lib().vxo_weight_numel(self._h, name.encode())
        p = lib().vxo_weight(self._h, name.encode())
        if not n or not p:
            raise KeyError(name)
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_uint16)), (n,))

    @property
    def is_ready(self):
        return bool(lib().vxo_is_ready(self._h))

    @property
    def position(self):
        return lib().vxo_position(self._h)

    @position.setter
    def position(self, p):
        lib().vxo_set_position(self._h, p)

    def reset(self):
        lib().vxo_reset(self._h)

    def set_kv_f16(self, on=True):
        """Store new K/V rows rounded to f16 (the engine's KV precision)."""
        lib().vxo_set_kv_f16(self._h, int(bool(on)))

    def buffer(self, name):
        n = c_int(0)
        p = lib().vxo_buffer(self._h, name.encode(), ctypes.byref(n))
        if not p:
            raise KeyError(name)
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_float)), (n.value,))

    def kv(self, layer, which):
        p = lib().vxo_kv(self._h, layer, which)
        kvd = self.cfg.n_kv_heads * self.cfg.head_dim
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_float)), (self.max_seq, kvd))

    @property
    def acoustic_codes(self):
        p = lib().vxo_acoustic_codes(self._h)
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_uint32)),
                                     (self.cfg.n_acoustic_out,)).copy()

    @acoustic_codes.setter
    def acoustic_codes(self, codes):
        lib().vxo_set_acoustic_codes(self._h, np.ascontiguousarray(codes, np.uint32))

    @property
    def semantic_code(self):
        return int(lib().vxo_semantic_argmax(self._h))

    @semantic_code.setter
    def semantic_code(self, c):
        lib().vxo_set_semantic_code(self._h, int(c))

    @property
    def argmax_result(self):
        return int(lib().vxo_argmax_result(self._h))

    def backbone_step(self, token=0, mode=0, precomputed=None, lm_head=False, layer_out=False):
        pre = None
        if precomputed is not None:
            pre = np.ascontiguousarray(precomputed, np.float32)
            mode = 2
        lo = None
        if layer_out:
            lo = np.empty((self.cfg.n_layers, 2, self.cfg.dim), np.float32)
        lib().vxo_backbone_step_ex(self._h, int(token), int(mode),
                                   pre.ctypes.data if pre is not None else None,
                                   int(bool(lm_head)),
                                   lo.ctypes.data if lo is not None else None)
        return lo

    def backbone_layer_by_layer(self, token=0, mode=0, precomputed=None):
        """debugBackboneLayerByLayer read points (src/engine.ts:2106-2287):
        embed and, per layer, attn_norm, attn_out, ffn_norm, ffn_out."""
        pre = None
        if precomputed is not None:
            pre = np.ascontiguousarray(precomputed, np.float32)
            mode = 2
        d = self.cfg.dim
        emb = np.empty(d, np.float32)
        lay = np.empty((self.cfg.n_layers, 4, d), np.float32)
        lib().vxo_backbone_step_debug(self._h, int(token), int(mode),
                                      pre.ctypes.data if pre is not None else None,
                                      emb.ctypes.data, lay.ctypes.data)
        names = ("attn_norm", "attn_out", "ffn_norm", "ffn_out")
        return {"embed": emb,
                "layers": [{n: lay[i, k] for k, n in enumerate(names)} for i in range(self.cfg.n_layers)],
                "final_norm": self.buffer("normed").copy(), "hidden": lay[-1, 3].copy()}

    def backbone_step_codes(self):
        lib().vxo_backbone_step_codes(self._h)

    def fm_forward(self, noise, batched=False):
        noise = np.ascontiguousarray(noise, np.float32)
        (lib().vxo_fm_forward_batched if batched else lib().vxo_fm_forward)(self._h, noise)

    def generate(self, tokens, audio_token_start, audio_token_count, voice_embeddings,
                 max_frames, noise_seed=0, ignore_eos=False, forced_semantic=None,
                 forced_acoustic=None, want_normed=False, want_logits=False):
        """generate() up to the codec decode (src/engine.ts:2416-2585): greedy
        masked semantic codes, FM noise from the engine's seeded fm.noise
        stream.  forced_semantic [n] / forced_acoustic [n][36]: the state
        each of the first n frames hands to the next (teacher forcing).
        Returns a dict of the per-frame outputs for every frame computed,
        including an EOS frame (framesGenerated = "frames")."""
        c = self.cfg
        toks = np.ascontiguousarray(tokens, np.int32)
        voice = None
        if voice_embeddings is not None:
            voice = np.ascontiguousarray(voice_embeddings, np.float32).ravel()
            if voice.size < audio_token_count * c.dim:
                raise ValueError("voice embeddings shorter than audio_token_count rows")
        n = max_frames
        sem = np.zeros(n, np.uint32)
        ac = np.zeros((n, c.n_acoustic_out), np.uint32)
        xt = np.zeros((n, c.n_acoustic_out), np.float32)
        normed = np.zeros((n, c.dim), np.float32) if want_normed else None
        logits = np.zeros((n, c.semantic_vocab), np.float32) if want_logits else None
        fs = fa = None
        nf = 0
        if forced_semantic is not None:
            fs = np.ascontiguousarray(forced_semantic, np.uint32)
            fa = np.ascontiguousarray(forced_acoustic, np.uint32).reshape(-1, c.n_acoustic_out)
            nf = min(fs.size, fa.shape[0])
        ptr = lambda a: a.ctypes.data if a is not None else None
        frames = lib().vxo_generate(self._h, ptr(toks), toks.size, int(audio_token_start),
                                    int(audio_token_count), ptr(voice), n, noise_seed,
                                    int(bool(ignore_eos)), ptr(fs), ptr(fa), nf, ptr(sem),
                                    ptr(ac), ptr(xt), ptr(normed), ptr(logits))
        if frames < 0:
            raise ValueError("prompt + frames exceed max_seq")
        m = min(frames + 1, n)  # the EOS frame's outputs too, when computed
        out = {"frames": frames, "semantic": sem[:m], "acoustic": ac[:m], "x_t": xt[:m]}
        if want_normed:
            out["normed"] = normed[:m]
        if want_logits:
            out["logits"] = logits[:m]
        return out


# ---------------------------------------------------------- codec decoder
CODEC_STOPS = ["concat", "after_input_conv",
               "after_stage0_transformer", "after_stage0_conv_up",
               "after_stage1_transformer", "after_stage1_conv_up",
               "after_stage2_transformer", "after_stage2_conv_up",
               "after_stage3_transformer", "audio"]


class OracleCodec:
    """CPU restatement of codecDecode (src/engine.ts:1402-1713) with the
    codec weights by name (src/engine.ts:700-770)."""

    def __init__(self):
        self._h = lib().vxo_codec_create()
        self._keep = {}

    def close(self):
        if self._h:
            lib().vxo_codec_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def names(self):
        L = lib()
        return [L.vxo_codec_weight_name(self._h, i).decode()
                for i in range(L.vxo_codec_n_weights(self._h))]

    def init_synthetic(self, seed=0, std=0.02):
        if lib().vxo_codec_init_synthetic(self._h, seed, std) != 0:
            raise MemoryError("oracle codec weights")

    def set_weight(self, name, bits):
        bits = np.ascontiguousarray(bits, np.uint16).ravel()
        if bits.size != lib().vxo_codec_weight_numel(self._h, name.encode()):
            raise ValueError(f"bad size for {name}")
        self._keep[name] = bits
        if lib().vxo_codec_set_weight(self._h, name.encode(), bits) != 0:
            raise KeyError(name)

    def weight(self, name):
        n = lib().vxo_codec_weight_numel(self._h, name.encode())
        p = lib().vxo_codec_weight(self._h, name.encode())
        if not n or not p:
            raise KeyError(name)
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_uint16)), (n,))

    def decode(self, semantic, acoustic, stop="audio"):
        """codecDecode up to a debugCodecDecode intermediate (default the
        waveform); semantic [T], acoustic [T][36]."""
        sem = np.ascontiguousarray(semantic, np.uint32).ravel()
        ac = np.ascontiguousarray(acoustic, np.uint32).ravel()
        T = sem.size
        if ac.size != 36 * T:
            raise ValueError("acoustic codes must be [T][36]")
        k = CODEC_STOPS.index(stop)
        out = np.empty(lib().vxo_codec_stop_count(T, k), np.float32)
        rc = lib().vxo_codec_decode(self._h, sem, ac, T, k, out)
        if rc != 0:
            raise RuntimeError(f"vxo_codec_decode failed ({rc})")
        return out

    def decode_all(self, semantic, acoustic):
        """every debugCodecDecode intermediate by name, in one pass"""
        sem = np.ascontiguousarray(semantic, np.uint32).ravel()
        ac = np.ascontiguousarray(acoustic, np.uint32).ravel()
        T = sem.size
        if ac.size != 36 * T:
            raise ValueError("acoustic codes must be [T][36]")
        outs = [np.empty(lib().vxo_codec_stop_count(T, k), np.float32) for k in range(10)]
        ptrs = (ctypes.c_void_p * 10)(*[o.ctypes.data for o in outs])
        rc = lib().vxo_codec_decode_all(self._h, sem, ac, T, ctypes.cast(ptrs, ctypes.c_void_p))
        if rc != 0:
            raise RuntimeError(f"vxo_codec_decode_all failed ({rc})")
        return dict(zip(CODEC_STOPS, outs))
