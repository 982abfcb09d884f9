// voxtral_napi.cc -- Node-API addon over the C ABI of libvoxtral_amd.so
// (include/voxtral_engine.h).  It is the binding the reference's TypeScript
// VoxtralEngine (src/engine.ts:291-2632) needs to run its per-frame token
// loop on the HIP engine: plain N-API (version 8 headers, Node >= 12), one
// native handle per engine, errors thrown as JS Error with the library's
// message, generate() on an async worker with onFrame/onStage marshalled
// back to the JS thread through thread-safe functions.
#include <node_api.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/voxtral_engine.h"

namespace {

#define NAPI_OK(env, call)                                       \
  do {                                                           \
    if ((call) != napi_ok) {                                     \
      napi_throw_error((env), nullptr, "N-API call failed: " #call); \
      return nullptr;                                            \
    }                                                            \
  } while (0)

napi_value throw_vx(napi_env env, vx_engine *e, int rc) {
  const char *m = vx_last_error(e);
  std::string msg = (m && *m) ? m : ("voxtral error " + std::to_string(rc));
  napi_throw_error(env, nullptr, msg.c_str());
  return nullptr;
}

struct Args {
  napi_value v[12];
  size_t n = 12;
};
bool get_args(napi_env env, napi_callback_info info, Args &a) {
  return napi_get_cb_info(env, info, &a.n, a.v, nullptr, nullptr) == napi_ok;
}

bool is_nullish(napi_env env, napi_value v) {
  napi_valuetype t;
  napi_typeof(env, v, &t);
  return t == napi_null || t == napi_undefined;
}

// One engine handle: the C-ABI engine and the state of a pending generate().
// A vx_engine serves one caller at a time and generate() runs on a worker
// thread, so while a generate() is in flight every other call on the handle
// throws (a second generate() rejects), and destroy() only marks the handle:
// the engine is freed when the pending generate() has completed.  A handle
// that is garbage-collected without destroy() frees its engine then.
struct EngineHandle {
  vx_engine *e = nullptr;
  bool busy = false;       // a generate() is running on the worker thread
  bool destroyed = false;  // destroy() was called
  int n_layers = 0;        // backbone layers of the engine's config
};

void handle_finalize(napi_env, void *data, void *) {
  auto *h = static_cast<EngineHandle *>(data);
  if (h->e && !h->busy) vx_destroy(h->e);
  delete h;
}

EngineHandle *handle_of(napi_env env, napi_value v) {
  void *p = nullptr;
  if (napi_get_value_external(env, v, &p) != napi_ok || !p) {
    napi_throw_type_error(env, nullptr, "invalid engine handle");
    return nullptr;
  }
  auto *h = static_cast<EngineHandle *>(p);
  if (h->destroyed) {
    napi_throw_error(env, nullptr, "engine destroyed");
    return nullptr;
  }
  return h;
}

// the engine behind a handle, for a call that must not overlap generate()
vx_engine *handle(napi_env env, napi_value v) {
  EngineHandle *h = handle_of(env, v);
  if (!h) return nullptr;
  if (h->busy) {
    napi_throw_error(env, nullptr, "generate() is still running on this engine");
    return nullptr;
  }
  return h->e;
}

double num(napi_env env, napi_value v, double dflt = 0) {
  double d = dflt;
  if (!is_nullish(env, v)) napi_get_value_double(env, v, &d);
  return d;
}

// a JS number that must be an integer in [lo, hi] (NaN, infinities, fractions
// and out-of-range values throw a RangeError naming `what`); null/undefined
// give dflt
bool int_arg(napi_env env, napi_value v, double lo, double hi, const char *what, double dflt,
             double *out) {
  double d = dflt;
  if (!is_nullish(env, v) && napi_get_value_double(env, v, &d) != napi_ok) {
    napi_throw_type_error(env, nullptr, (std::string(what) + " must be a number").c_str());
    return false;
  }
  if (!std::isfinite(d) || d != std::floor(d) || d < lo || d > hi) {
    napi_throw_range_error(env, nullptr, (std::string(what) + " out of range").c_str());
    return false;
  }
  *out = d;
  return true;
}
constexpr double kI32Min = -2147483648.0, kI32Max = 2147483647.0, kU32Max = 4294967295.0;
// seeds: integers in [0, 2^64)
constexpr double kU64Lim = 18446744073709549568.0;  // largest double below 2^64

std::string str(napi_env env, napi_value v) {
  size_t n = 0;
  napi_get_value_string_utf8(env, v, nullptr, 0, &n);
  std::string s(n, '\0');
  napi_get_value_string_utf8(env, v, &s[0], n + 1, &n);
  return s;
}

// typed array data of the expected element type, or nullptr (and a thrown
// TypeError) on mismatch
void *typed(napi_env env, napi_value v, napi_typedarray_type want, size_t *len) {
  bool ok = false;
  napi_is_typedarray(env, v, &ok);
  napi_typedarray_type t;
  void *data = nullptr;
  napi_value ab;
  size_t off = 0;
  if (!ok || napi_get_typedarray_info(env, v, &t, len, &data, &ab, &off) != napi_ok || t != want) {
    napi_throw_type_error(env, nullptr, "unexpected typed array type");
    return nullptr;
  }
  return data;
}

napi_value new_f32(napi_env env, const float *src, size_t n) {
  void *data = nullptr;
  napi_value ab, out;
  if (napi_create_arraybuffer(env, n * 4, &data, &ab) != napi_ok) return nullptr;
  if (n) memcpy(data, src, n * 4);
  napi_create_typedarray(env, napi_float32_array, n, ab, 0, &out);
  return out;
}
napi_value new_u32(napi_env env, const uint32_t *src, size_t n) {
  void *data = nullptr;
  napi_value ab, out;
  if (napi_create_arraybuffer(env, n * 4, &data, &ab) != napi_ok) return nullptr;
  if (n) memcpy(data, src, n * 4);
  napi_create_typedarray(env, napi_uint32_array, n, ab, 0, &out);
  return out;
}

void set_int(napi_env env, napi_value obj, const char *k, double v) {
  napi_value x;
  napi_create_double(env, v, &x);
  napi_set_named_property(env, obj, k, x);
}

// ------------------------------------------------------------ lifecycle
// create(config | null, maxSeqLen) -> handle.  config: partial object of
// vx_config fields in the reference's camelCase (src/types.ts:70-122).
napi_value create(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a)) return nullptr;
  vx_config c;
  vx_config_default(&c);
  if (a.n > 0 && !is_nullish(env, a.v[0])) {
    struct F {
      const char *k;
      int32_t *i;
      float *f;
    } fields[] = {{"dim", &c.dim, nullptr},
                  {"nLayers", &c.n_layers, nullptr},
                  {"headDim", &c.head_dim, nullptr},
                  {"hiddenDim", &c.hidden_dim, nullptr},
                  {"nHeads", &c.n_heads, nullptr},
                  {"nKvHeads", &c.n_kv_heads, nullptr},
                  {"vocabSize", &c.vocab_size, nullptr},
                  {"ropeTheta", nullptr, &c.rope_theta},
                  {"normEps", nullptr, &c.norm_eps},
                  {"fmLayers", &c.fm_layers, nullptr},
                  {"nfe", &c.nfe, nullptr},
                  {"cfgAlpha", nullptr, &c.cfg_alpha},
                  {"kvF16", &c.kv_f16, nullptr},
                  {"codec", &c.codec, nullptr}};
    for (auto &f : fields) {
      bool has = false;
      napi_has_named_property(env, a.v[0], f.k, &has);
      if (!has) continue;
      napi_value v;
      napi_get_named_property(env, a.v[0], f.k, &v);
      if (f.i) {
        double d = 0;
        if (!int_arg(env, v, kI32Min, kI32Max, f.k, 0, &d)) return nullptr;
        *f.i = (int32_t)d;
      } else {
        *f.f = (float)num(env, v);
      }
    }
  }
  double ms = 4096;
  if (a.n > 1 && !int_arg(env, a.v[1], kI32Min, kI32Max, "maxSeqLen", 4096, &ms)) return nullptr;
  vx_engine *e = nullptr;
  int rc = vx_create(&c, (int32_t)ms, &e);
  if (rc) return throw_vx(env, nullptr, rc);
  auto *eh = new EngineHandle();
  eh->e = e;
  eh->n_layers = c.n_layers;
  napi_value h;
  if (napi_create_external(env, eh, handle_finalize, nullptr, &h) != napi_ok) {
    vx_destroy(e);
    delete eh;
    napi_throw_error(env, nullptr, "N-API call failed: napi_create_external");
    return nullptr;
  }
  return h;
}

// destroy(h): frees the engine now, or, while a generate() is running, as
// soon as it completes; the handle is unusable from here on
napi_value destroy(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a) || a.n < 1) return nullptr;
  void *p = nullptr;
  if (napi_get_value_external(env, a.v[0], &p) != napi_ok || !p) {
    napi_throw_type_error(env, nullptr, "invalid engine handle");
    return nullptr;
  }
  auto *h = static_cast<EngineHandle *>(p);
  if (h->destroyed) return nullptr;
  h->destroyed = true;
  if (!h->busy && h->e) {
    vx_destroy(h->e);
    h->e = nullptr;
  }
  return nullptr;
}

// loadTensor(h, name, Uint16Array f16, shape number[])
napi_value load_tensor(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a) || a.n < 4) return nullptr;
  vx_engine *e = handle(env, a.v[0]);
  if (!e) return nullptr;
  std::string name = str(env, a.v[1]);
  size_t n = 0;
  auto *data = (const uint16_t *)typed(env, a.v[2], napi_uint16_array, &n);
  if (!data) return nullptr;
  uint32_t nd = 0;
  napi_get_array_length(env, a.v[3], &nd);
  std::vector<int64_t> shape(nd);
  for (uint32_t i = 0; i < nd; i++) {
    napi_value x;
    napi_get_element(env, a.v[3], i, &x);
    double d = 0;
    if (!int_arg(env, x, 0, 9007199254740991.0, "shape", 0, &d)) return nullptr;
    shape[i] = (int64_t)d;
  }
  int rc = vx_load_tensor(e, name.c_str(), data, n, shape.data(), (int32_t)nd);
  if (rc) return throw_vx(env, e, rc);
  return nullptr;
}

// loadSafetensors(h, path[, onTensor]) -> {loaded, skipped}.  onTensor(loaded,
// total, component, tensor, bytesRead) is called on this thread after each
// tensor reaches the device; once it throws, it is not called again and the
// exception propagates when the load returns.
struct LoadProgress {
  napi_env env;
  napi_value fn;
  bool failed;
};
static void load_progress(void *user, int32_t loaded, int32_t total, const char *component,
                          const char *tensor, uint64_t bytes) {
  auto *p = (LoadProgress *)user;
  if (p->failed) return;
  napi_value args[5], global, ret;
  napi_create_int32(p->env, loaded, &args[0]);
  napi_create_int32(p->env, total, &args[1]);
  napi_create_string_utf8(p->env, component, NAPI_AUTO_LENGTH, &args[2]);
  napi_create_string_utf8(p->env, tensor, NAPI_AUTO_LENGTH, &args[3]);
  napi_create_double(p->env, (double)bytes, &args[4]);
  napi_get_global(p->env, &global);
  if (napi_call_function(p->env, global, p->fn, 5, args, &ret) != napi_ok) p->failed = true;
  bool pending = false;
  napi_is_exception_pending(p->env, &pending);
  if (pending) p->failed = true;
}

napi_value load_safetensors(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a) || a.n < 2) return nullptr;
  vx_engine *e = handle(env, a.v[0]);
  if (!e) return nullptr;
  std::string path = str(env, a.v[1]);
  LoadProgress prog{env, nullptr, false};
  if (a.n > 2 && !is_nullish(env, a.v[2])) {
    napi_valuetype t;
    napi_typeof(env, a.v[2], &t);
    if (t != napi_function) {
      napi_throw_type_error(env, nullptr, "onTensor must be a function");
      return nullptr;
    }
    prog.fn = a.v[2];
  }
  int32_t loaded = 0, skipped = 0;
  int rc = vx_load_safetensors_progress(e, path.c_str(), prog.fn ? load_progress : nullptr, &prog,
                                        &loaded, &skipped);
  bool pending = false;
  napi_is_exception_pending(env, &pending);
  if (pending) return nullptr;
  if (rc) return throw_vx(env, e, rc);
  napi_value o, x;
  NAPI_OK(env, napi_create_object(env, &o));
  NAPI_OK(env, napi_create_int32(env, loaded, &x));
  NAPI_OK(env, napi_set_named_property(env, o, "loaded", x));
  NAPI_OK(env, napi_create_int32(env, skipped, &x));
  NAPI_OK(env, napi_set_named_property(env, o, "skipped", x));
  return o;
}

// missingTensor(h) -> the first weight not loaded yet, or null
napi_value missing_tensor(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a) || a.n < 1) return nullptr;
  vx_engine *e = handle(env, a.v[0]);
  if (!e) return nullptr;
  char name[512];
  napi_value r;
  if (vx_missing_tensor(e, name, (int32_t)sizeof name)) {
    napi_create_string_utf8(env, name, NAPI_AUTO_LENGTH, &r);
  } else {
    napi_get_null(env, &r);
  }
  return r;
}

// codecDecode(h, Uint32Array semantic, Uint32Array acoustic[, stop]) ->
// Float32Array (stop: VX_CODEC_STOP_*, default the waveform)
napi_value codec_decode(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a) || a.n < 3) return nullptr;
  vx_engine *e = handle(env, a.v[0]);
  if (!e) return nullptr;
  size_t ns = 0, na = 0;
  auto *sem = (const uint32_t *)typed(env, a.v[1], napi_uint32_array, &ns);
  if (!sem) return nullptr;
  auto *ac = (const uint32_t *)typed(env, a.v[2], napi_uint32_array, &na);
  if (!ac) return nullptr;
  if (na != ns * 36) {
    napi_throw_range_error(env, nullptr, "acousticCodes must hold 36 codes per frame");
    return nullptr;
  }
  double sd = VX_CODEC_STOP_AUDIO;
  if (a.n > 3 && !int_arg(env, a.v[3], kI32Min, kI32Max, "stop", VX_CODEC_STOP_AUDIO, &sd))
    return nullptr;
  const int32_t stop = (int32_t)sd;
  std::vector<float> out(std::max<size_t>(vx_codec_stop_count((int32_t)ns, stop), 1));
  int rc = vx_codec_decode_debug(e, sem, ac, (int32_t)ns, stop, out.data(), out.size());
  if (rc) return throw_vx(env, e, rc);
  return new_f32(env, out.data(), vx_codec_stop_count((int32_t)ns, stop));
}

// ------------------------------------------------------------ tokenizer
void tokenizer_finalize(napi_env, void *data, void *) {
  vx_tokenizer_destroy(static_cast<vx_tokenizer *>(data));
}

// tokenizerCreate(Uint8Array blob, Int32Array offsets[n + 1], Int32Array ranks[n],
//                 numSpecial) -> external (freed with the JS object)
napi_value tokenizer_create(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a) || a.n < 4) return nullptr;
  size_t nb = 0, no = 0, nr = 0;
  auto *blob = (const uint8_t *)typed(env, a.v[0], napi_uint8_array, &nb);
  auto *off = (const int32_t *)typed(env, a.v[1], napi_int32_array, &no);
  auto *ranks = (const int32_t *)typed(env, a.v[2], napi_int32_array, &nr);
  if (!blob || !off || !ranks) return nullptr;
  if (no != nr + 1 || (size_t)off[nr] > nb) {
    napi_throw_range_error(env, nullptr, "tokenizer vocabulary arrays do not match");
    return nullptr;
  }
  std::vector<int64_t> off64(off, off + no);
  vx_tokenizer *t = nullptr;
  double ns = 0;
  if (!int_arg(env, a.v[3], 0, kI32Max, "numSpecial", 0, &ns)) return nullptr;
  int rc = vx_tokenizer_create(blob, off64.data(), ranks, (int32_t)nr, (int32_t)ns, &t);
  if (rc) return throw_vx(env, nullptr, rc);
  napi_value h;
  NAPI_OK(env, napi_create_external(env, t, tokenizer_finalize, nullptr, &h));
  return h;
}

// tokenizerEncode(handle, Uint8Array bytes, Int32Array offsets[n + 1]) -> Int32Array
napi_value tokenizer_encode(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a) || a.n < 3) return nullptr;
  void *p = nullptr;
  if (napi_get_value_external(env, a.v[0], &p) != napi_ok || !p) {
    napi_throw_type_error(env, nullptr, "not a tokenizer handle");
    return nullptr;
  }
  size_t nb = 0, no = 0;
  auto *bytes = (const uint8_t *)typed(env, a.v[1], napi_uint8_array, &nb);
  auto *off = (const int32_t *)typed(env, a.v[2], napi_int32_array, &no);
  if (!bytes || !off) return nullptr;
  if (no < 1 || (size_t)off[no - 1] > nb) {
    napi_throw_range_error(env, nullptr, "piece offsets do not match the bytes");
    return nullptr;
  }
  std::vector<int64_t> off64(off, off + no);
  const int64_t cap = (int64_t)nb + (int64_t)no;
  std::vector<int32_t> ids((size_t)cap);
  int64_t n = 0;
  int rc = vx_tokenizer_encode_pieces(static_cast<vx_tokenizer *>(p), bytes, off64.data(),
                                      (int32_t)(no - 1), ids.data(), cap, &n);
  if (rc) return throw_vx(env, nullptr, rc);
  napi_value ab, out;
  void *dst = nullptr;
  NAPI_OK(env, napi_create_arraybuffer(env, (size_t)n * 4, &dst, &ab));
  if (n) memcpy(dst, ids.data(), (size_t)n * 4);
  NAPI_OK(env, napi_create_typedarray(env, napi_int32_array, (size_t)n, ab, 0, &out));
  return out;
}

napi_value init_synthetic(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a) || a.n < 3) return nullptr;
  vx_engine *e = handle(env, a.v[0]);
  if (!e) return nullptr;
  double seed = 0;
  if (!int_arg(env, a.v[1], 0, kU64Lim, "seed", 0, &seed)) return nullptr;
  int rc = vx_init_synthetic(e, (uint64_t)seed, (float)num(env, a.v[2], 0.02));
  if (rc) return throw_vx(env, e, rc);
  return nullptr;
}

napi_value is_ready(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a) || a.n < 1) return nullptr;
  EngineHandle *h = handle_of(env, a.v[0]);  // weight flags only: fine during generate()
  if (!h) return nullptr;
  vx_engine *e = h->e;
  napi_value b;
  napi_get_boolean(env, vx_is_ready(e) != 0, &b);
  return b;
}

napi_value reset(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a) || a.n < 1) return nullptr;
  vx_engine *e = handle(env, a.v[0]);
  if (!e) return nullptr;
  int rc = vx_reset(e);
  if (rc) return throw_vx(env, e, rc);
  return nullptr;
}

napi_value position(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a) || a.n < 1) return nullptr;
  vx_engine *e = handle(env, a.v[0]);
  if (!e) return nullptr;
  if (a.n > 1 && !is_nullish(env, a.v[1])) {
    double p = 0;
    if (!int_arg(env, a.v[1], kI32Min, kI32Max, "position", 0, &p)) return nullptr;
    int rc = vx_set_position(e, (int32_t)p);
    if (rc) return throw_vx(env, e, rc);
  }
  napi_value v;
  napi_create_int32(env, vx_position(e), &v);
  return v;
}

// ------------------------------------------------------------ steps
// backboneStep(h, token, embedMode, precomputed Float32Array|null, lmHead)
//   -> {argmax, normed: Float32Array}
napi_value backbone_step(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a) || a.n < 5) return nullptr;
  vx_engine *e = handle(env, a.v[0]);
  if (!e) return nullptr;
  const float *pre = nullptr;
  if (!is_nullish(env, a.v[3])) {
    size_t n = 0;
    pre = (const float *)typed(env, a.v[3], napi_float32_array, &n);
    if (!pre) return nullptr;
    if (n < 3072) {
      napi_throw_range_error(env, nullptr, "precomputed embedding needs 3072 values");
      return nullptr;
    }
  }
  bool lm = false;
  napi_get_value_bool(env, a.v[4], &lm);
  uint32_t am = 0;
  std::vector<float> normed(3072);
  double tok = 0, mode = 0;
  if (!int_arg(env, a.v[1], kI32Min, kI32Max, "tokenId", 0, &tok) ||
      !int_arg(env, a.v[2], kI32Min, kI32Max, "embedMode", 0, &mode))
    return nullptr;
  int rc = vx_backbone_step(e, (int32_t)tok, (int32_t)mode, pre, lm ? 1 : 0,
                            &am, normed.data());
  if (rc) return throw_vx(env, e, rc);
  napi_value out;
  napi_create_object(env, &out);
  set_int(env, out, "argmax", am);
  napi_set_named_property(env, out, "normed", new_f32(env, normed.data(), normed.size()));
  return out;
}

// backboneLayers(h, token, embedMode, precomputed Float32Array|null)
//   -> {embed: Float32Array(3072), layers: Float32Array(nLayers * 4 * 3072)}
// (per layer attn_norm, attn_out, ffn_norm, ffn_out: the read points of
// debugBackboneLayerByLayer)
napi_value backbone_layers(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a) || a.n < 4) return nullptr;
  EngineHandle *h = handle_of(env, a.v[0]);
  if (!h) return nullptr;
  vx_engine *e = handle(env, a.v[0]);
  if (!e) return nullptr;
  const float *pre = nullptr;
  if (!is_nullish(env, a.v[3])) {
    size_t n = 0;
    pre = (const float *)typed(env, a.v[3], napi_float32_array, &n);
    if (!pre) return nullptr;
    if (n < 3072) {
      napi_throw_range_error(env, nullptr, "precomputed embedding needs 3072 values");
      return nullptr;
    }
  }
  double tok = 0, mode = 0;
  if (!int_arg(env, a.v[1], kI32Min, kI32Max, "tokenId", 0, &tok) ||
      !int_arg(env, a.v[2], kI32Min, kI32Max, "embedMode", 0, &mode))
    return nullptr;
  std::vector<float> embed(3072), layers((size_t)h->n_layers * 4 * 3072);
  int rc = vx_debug_backbone_layers(e, (int32_t)tok, (int32_t)mode, pre, embed.data(), layers.data());
  if (rc) return throw_vx(env, e, rc);
  napi_value out;
  napi_create_object(env, &out);
  napi_set_named_property(env, out, "embed", new_f32(env, embed.data(), embed.size()));
  napi_set_named_property(env, out, "layers", new_f32(env, layers.data(), layers.size()));
  return out;
}

// fmForward(h, noise Float32Array(36)|null)
//   -> {semanticLogits: Float32Array, acousticCodes: Uint32Array, xFinal}
napi_value fm_forward(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a) || a.n < 2) return nullptr;
  vx_engine *e = handle(env, a.v[0]);
  if (!e) return nullptr;
  const float *noise = nullptr;
  if (!is_nullish(env, a.v[1])) {
    size_t n = 0;
    noise = (const float *)typed(env, a.v[1], napi_float32_array, &n);
    if (!noise) return nullptr;
    if (n < 36) {
      napi_throw_range_error(env, nullptr, "noise needs 36 values");
      return nullptr;
    }
  }
  std::vector<float> logits(8320), xf(36);
  uint32_t codes[36];
  int rc = vx_fm_forward(e, noise, logits.data(), codes, xf.data());
  if (rc) return throw_vx(env, e, rc);
  napi_value out;
  napi_create_object(env, &out);
  napi_set_named_property(env, out, "semanticLogits", new_f32(env, logits.data(), logits.size()));
  napi_set_named_property(env, out, "acousticCodes", new_u32(env, codes, 36));
  napi_set_named_property(env, out, "xFinal", new_f32(env, xf.data(), xf.size()));
  return out;
}

napi_value set_semantic_code(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a) || a.n < 2) return nullptr;
  vx_engine *e = handle(env, a.v[0]);
  if (!e) return nullptr;
  double code = 0;
  if (!int_arg(env, a.v[1], 0, kU32Max, "semanticCode", 0, &code)) return nullptr;
  int rc = vx_set_semantic_code(e, (uint32_t)code);
  if (rc) return throw_vx(env, e, rc);
  return nullptr;
}

// read(h, name, count) -> Float32Array
napi_value read(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a) || a.n < 3) return nullptr;
  vx_engine *e = handle(env, a.v[0]);
  if (!e) return nullptr;
  std::string name = str(env, a.v[1]);
  double cnt = 16;
  if (!int_arg(env, a.v[2], 0, 1 << 28, "count", 16, &cnt)) return nullptr;
  std::vector<float> buf((size_t)cnt);
  int rc = vx_read(e, name.c_str(), buf.data(), buf.size());
  if (rc) return throw_vx(env, e, rc);
  return new_f32(env, buf.data(), buf.size());
}

// ------------------------------------------------------------ generate
// Frames, stage marks and the final result travel through one thread-safe
// function, whose queue is FIFO: every onFrame/onStage call reaches the JS
// thread before the promise settles, as in the reference, where they run
// synchronously inside generate() (src/engine.ts:2584).
enum MsgKind { MSG_FRAME, MSG_STAGE, MSG_DONE };
struct Msg {
  MsgKind kind;
  int32_t frame;
  uint32_t semantic;
  uint32_t codes[36];
  int32_t stage;
  double done_ms;
};

struct GenJob {
  vx_engine *e;
  EngineHandle *h;              // busy while the job runs
  napi_ref handle_ref = nullptr;  // keeps the handle alive until the job is done
  std::vector<int32_t> tokens;
  int32_t audio_start, audio_count, max_frames;
  std::vector<float> voice;
  bool has_voice;
  vx_generate_options opt;
  napi_ref on_frame = nullptr, on_stage = nullptr;
  napi_threadsafe_function events = nullptr;
  std::vector<uint32_t> sem, ac;
  bool want_audio = false;
  std::vector<float> audio;
  vx_generate_stats stats;
  int rc = 0;
  std::string err;
  napi_deferred deferred;
  napi_async_work work;
};

void settle(napi_env env, GenJob *j) {
  if (j->rc) {
    napi_value msg, err;
    napi_create_string_utf8(env, j->err.c_str(), NAPI_AUTO_LENGTH, &msg);
    napi_create_error(env, nullptr, msg, &err);
    napi_reject_deferred(env, j->deferred, err);
    return;
  }
  const int n = j->stats.frames_generated;
  napi_value out, sem, ac, stats;
  napi_create_object(env, &out);
  napi_create_array_with_length(env, n, &sem);
  napi_create_array_with_length(env, n, &ac);
  for (int f = 0; f < n; f++) {
    napi_value v, row;
    napi_create_uint32(env, j->sem[f], &v);
    napi_set_element(env, sem, f, v);
    napi_create_array_with_length(env, 36, &row);
    for (int k = 0; k < 36; k++) {
      napi_value c;
      napi_create_uint32(env, j->ac[(size_t)f * 36 + k], &c);
      napi_set_element(env, row, k, c);
    }
    napi_set_element(env, ac, f, row);
  }
  napi_set_named_property(env, out, "semanticCodes", sem);
  napi_set_named_property(env, out, "acousticCodes", ac);
  napi_set_named_property(env, out, "audio",
                          new_f32(env, j->audio.data(), j->want_audio ? (size_t)n * VX_FRAME_SAMPLES : 0));
  napi_create_object(env, &stats);
  set_int(env, stats, "backboneMs", j->stats.backbone_ms);
  set_int(env, stats, "fmMs", j->stats.fm_ms);
  set_int(env, stats, "codecMs", j->stats.codec_ms);
  set_int(env, stats, "totalMs", j->stats.total_ms);
  set_int(env, stats, "framesGenerated", n);
  napi_set_named_property(env, out, "stats", stats);
  napi_resolve_deferred(env, j->deferred, out);
}

// runs on the JS thread, in queue order
void dispatch(napi_env env, napi_value, void *context, void *data) {
  auto *j = static_cast<GenJob *>(context);
  auto *m = static_cast<Msg *>(data);
  if (env) {
    napi_value undef, cb;
    napi_get_undefined(env, &undef);
    if (m->kind == MSG_FRAME && j->on_frame &&
        napi_get_reference_value(env, j->on_frame, &cb) == napi_ok) {
      napi_value argv[3];
      napi_create_int32(env, m->frame, &argv[0]);
      napi_create_uint32(env, m->semantic, &argv[1]);
      argv[2] = new_u32(env, m->codes, 36);
      napi_call_function(env, undef, cb, 3, argv, nullptr);
    } else if (m->kind == MSG_STAGE && j->on_stage &&
               napi_get_reference_value(env, j->on_stage, &cb) == napi_ok) {
      static const char *names[] = {"backbone", "fm", "codec"};
      napi_value argv[2];
      napi_create_string_utf8(env, names[m->stage < 0 || m->stage > 2 ? 0 : m->stage],
                              NAPI_AUTO_LENGTH, &argv[0]);
      if (m->done_ms < 0) napi_get_undefined(env, &argv[1]);
      else napi_create_double(env, m->done_ms, &argv[1]);
      napi_call_function(env, undef, cb, 2, argv, nullptr);
    } else if (m->kind == MSG_DONE) {
      // the engine is free again before the promise's continuations run; a
      // destroy() that arrived meanwhile frees it now
      j->h->busy = false;
      if (j->h->destroyed && j->h->e) {
        vx_destroy(j->h->e);
        j->h->e = nullptr;
      }
      settle(env, j);
      if (j->on_frame) napi_delete_reference(env, j->on_frame);
      if (j->on_stage) napi_delete_reference(env, j->on_stage);
      if (j->handle_ref) napi_delete_reference(env, j->handle_ref);
      napi_release_threadsafe_function(j->events, napi_tsfn_release);
      delete m;
      delete j;
      return;
    }
  }
  delete m;
}

void post(GenJob *j, Msg *m) {
  if (napi_call_threadsafe_function(j->events, m, napi_tsfn_blocking) != napi_ok) delete m;
}

void frame_cb(void *user, int32_t f, uint32_t s, const uint32_t *codes) {
  auto *j = static_cast<GenJob *>(user);
  if (!j->on_frame) return;
  auto *m = new Msg{MSG_FRAME, f, s, {}, 0, 0};
  memcpy(m->codes, codes, sizeof m->codes);
  post(j, m);
}

void stage_cb(void *user, int32_t st, double done) {
  auto *j = static_cast<GenJob *>(user);
  if (!j->on_stage) return;
  post(j, new Msg{MSG_STAGE, 0, 0, {}, st, done});
}

void gen_execute(napi_env, void *data) {
  auto *j = static_cast<GenJob *>(data);
  const int nf = j->max_frames > 0 ? j->max_frames : 1;
  j->sem.assign(nf, 0);
  j->ac.assign((size_t)nf * 36, 0);
  if (j->want_audio) j->audio.assign((size_t)nf * VX_FRAME_SAMPLES, 0.f);
  j->rc = vx_generate(j->e, j->tokens.data(), (int32_t)j->tokens.size(), j->audio_start,
                      j->audio_count, j->has_voice ? j->voice.data() : nullptr, j->max_frames,
                      &j->opt, frame_cb, stage_cb, j, j->sem.data(), j->ac.data(),
                      j->want_audio ? j->audio.data() : nullptr, &j->stats);
  if (j->rc) j->err = vx_last_error(j->e);
}

// JS thread, after gen_execute: the result goes behind every queued frame
void gen_complete(napi_env env, napi_status, void *data) {
  auto *j = static_cast<GenJob *>(data);
  napi_delete_async_work(env, j->work);
  post(j, new Msg{MSG_DONE, 0, 0, {}, 0, 0});
}

// generate(h, tokens number[]|Int32Array, audioTokenStart, audioTokenCount,
//          voice Float32Array|null, maxFrames, options|null, onFrame?, onStage?)
//   -> Promise<{semanticCodes, acousticCodes, stats}>
napi_value generate(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a) || a.n < 6) {
    napi_throw_type_error(env, nullptr, "generate needs at least 6 arguments");
    return nullptr;
  }
  vx_engine *e = handle(env, a.v[0]);  // throws while another generate() runs
  if (!e) return nullptr;
  auto *j = new GenJob();
  j->e = e;
  j->h = handle_of(env, a.v[0]);
  bool is_ta = false;
  napi_is_typedarray(env, a.v[1], &is_ta);
  if (is_ta) {
    size_t n = 0;
    auto *p = (const int32_t *)typed(env, a.v[1], napi_int32_array, &n);
    if (!p) {
      delete j;
      return nullptr;
    }
    j->tokens.assign(p, p + n);
  } else {
    uint32_t nt = 0;
    napi_get_array_length(env, a.v[1], &nt);
    j->tokens.resize(nt);
    for (uint32_t i = 0; i < nt; i++) {
      napi_value x;
      napi_get_element(env, a.v[1], i, &x);
      double t = 0;
      if (!int_arg(env, x, kI32Min, kI32Max, "token", 0, &t)) {
        delete j;
        return nullptr;
      }
      j->tokens[i] = (int32_t)t;
    }
  }
  double as = 0, ac = 0;
  if (!int_arg(env, a.v[2], kI32Min, kI32Max, "audioTokenStart", 0, &as) ||
      !int_arg(env, a.v[3], 0, kI32Max, "audioTokenCount", 0, &ac)) {
    delete j;
    return nullptr;
  }
  j->audio_start = (int32_t)as;
  j->audio_count = (int32_t)ac;
  j->has_voice = !is_nullish(env, a.v[4]);
  if (j->has_voice) {
    size_t n = 0;
    auto *p = (const float *)typed(env, a.v[4], napi_float32_array, &n);
    if (!p) {
      delete j;
      return nullptr;
    }
    j->voice.assign(p, p + n);
    if (j->audio_count > 0 && n < (size_t)j->audio_count * 3072) {
      delete j;
      napi_throw_range_error(env, nullptr, "voiceEmbeddings shorter than audioTokenCount rows");
      return nullptr;
    }
  }
  double mf = 500;
  if (!int_arg(env, a.v[5], 0, kI32Max, "maxFrames", 500, &mf)) {
    delete j;
    return nullptr;
  }
  j->max_frames = (int32_t)mf;
  vx_generate_options_default(&j->opt);
  if (a.n > 6 && !is_nullish(env, a.v[6])) {
    napi_value v;
    bool has = false;
    napi_has_named_property(env, a.v[6], "sampling", &has);
    if (has) {
      napi_get_named_property(env, a.v[6], "sampling", &v);
      const std::string m = str(env, v);
      if (m != "greedy" && m != "top_p" && m != "top_p_host") {
        delete j;
        napi_throw_range_error(env, nullptr, "sampling must be 'top_p', 'top_p_host' or 'greedy'");
        return nullptr;
      }
      j->opt.sampling = m == "greedy" ? VX_SAMPLE_GREEDY
                        : m == "top_p_host" ? VX_SAMPLE_TOP_P_HOST : VX_SAMPLE_TOP_P;
    }
    const char *keys[] = {"topP", "temperature", "seed", "ignoreEos", "audio"};
    for (int k = 0; k < 5; k++) {
      napi_has_named_property(env, a.v[6], keys[k], &has);
      if (!has) continue;
      napi_get_named_property(env, a.v[6], keys[k], &v);
      napi_valuetype t;
      napi_typeof(env, v, &t);
      double d = 0;
      if (t == napi_boolean) {
        bool b = false;
        napi_get_value_bool(env, v, &b);
        d = b;
      } else if (k == 2) {
        if (!int_arg(env, v, 0, kU64Lim, "seed", 0, &d)) {
          delete j;
          return nullptr;
        }
      } else {
        d = num(env, v);  // topP / temperature: the library rejects bad values
      }
      if (k == 0) j->opt.top_p = d;
      if (k == 1) j->opt.temperature = d;
      if (k == 2) j->opt.seed = (uint64_t)d;
      if (k == 3) j->opt.ignore_eos = d != 0;
      if (k == 4) j->want_audio = d != 0;
    }
  }
  if (a.n > 7 && !is_nullish(env, a.v[7])) napi_create_reference(env, a.v[7], 1, &j->on_frame);
  if (a.n > 8 && !is_nullish(env, a.v[8])) napi_create_reference(env, a.v[8], 1, &j->on_stage);
  napi_value name, promise;
  napi_create_string_utf8(env, "voxtral.generate", NAPI_AUTO_LENGTH, &name);
  if (napi_create_threadsafe_function(env, nullptr, nullptr, name, 0, 1, nullptr, nullptr, j,
                                      dispatch, &j->events) != napi_ok) {
    if (j->on_frame) napi_delete_reference(env, j->on_frame);
    if (j->on_stage) napi_delete_reference(env, j->on_stage);
    delete j;
    napi_throw_error(env, nullptr, "could not create the generate event queue");
    return nullptr;
  }
  napi_create_reference(env, a.v[0], 1, &j->handle_ref);
  j->h->busy = true;
  napi_create_promise(env, &j->deferred, &promise);
  napi_create_async_work(env, nullptr, name, gen_execute, gen_complete, j, &j->work);
  napi_queue_async_work(env, j->work);
  return promise;
}

napi_value init(napi_env env, napi_value exports) {
  struct {
    const char *name;
    napi_callback fn;
  } fns[] = {{"create", create},
             {"destroy", destroy},
             {"loadTensor", load_tensor},
             {"loadSafetensors", load_safetensors},
             {"codecDecode", codec_decode},
             {"tokenizerCreate", tokenizer_create},
             {"tokenizerEncode", tokenizer_encode},
             {"initSynthetic", init_synthetic},
             {"isReady", is_ready},
             {"missingTensor", missing_tensor},
             {"reset", reset},
             {"position", position},
             {"backboneStep", backbone_step},
             {"backboneLayers", backbone_layers},
             {"fmForward", fm_forward},
             {"setSemanticCode", set_semantic_code},
             {"read", read},
             {"generate", generate}};
  for (auto &f : fns) {
    napi_value v;
    napi_create_function(env, f.name, NAPI_AUTO_LENGTH, f.fn, nullptr, &v);
    napi_set_named_property(env, exports, f.name, v);
  }
  return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, init)
