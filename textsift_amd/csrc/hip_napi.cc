// hip_napi.cc — the Node-API module textsift's NodeBackend loads for the
// "hip" platform (textsift_amd/lib/textsift-hip.node).
//
// The reference's Node host reaches its native GPU backends through the
// NativeApi verbs (packages/textsift/src/native/backend.ts:34-131),
// implemented per platform as vulkan*/metal*/dawn* functions in
// native/napi.zig:546-864. This module registers the same verbs with a "hip"
// prefix over the C ABI in include/pfhip.h, plus the whole-forward and Viterbi
// entries the HIP backend adds:
//
//   hipCreateBackend([device]) -> BigInt          hipDestroyBackend(h)
//   hipDeviceName(h) -> string
//   hipCreateBuffer(h, Uint8Array) -> BigInt      hipCreateEmptyBuffer(h, n) -> BigInt
//   hipReleaseBuffer(h, buf)                      hipWriteBuffer(h, buf, offset, Uint8Array)
//   hipReadBuffer(h, buf, offset, n) -> Uint8Array
//   hipDispatchOneShot(h, name, BigInt[] bindings, Uint8Array push, [gx, gy, gz])
//   hipBeginEncoder(h) -> BigInt
//   hipEnqueueDispatch(enc, name, BigInt[] bindings, Uint8Array push, [gx, gy, gz])
//   hipSubmitAndReadback(enc, outBuf, offset, n) -> Uint8Array
//   hipKernelNames() -> string                    hipVersion() -> string
//   hipModelCreate(h, config) -> BigInt           hipModelDestroy(m)
//   hipModelSetWeight(m, name, Uint8Array)        hipModelFinalize(m)
//   hipForward(m, Int32Array ids, Uint8Array|null mask, batch, seqLen) -> Float32Array
//   hipViterbiDecode(Float32Array logits, batch, seqStride, Uint32Array|null seqLens,
//                    Float32Array biases[6], nThreads) -> Uint8Array
//
// Handles are native pointers carried as BigInt (0 is invalid), as in
// napi.zig. Every failure becomes a thrown JS Error carrying the library's
// message (napi.zig:64-67 napiThrow); nothing aborts the process. At most 16
// bindings per dispatch (napi.zig:716-739).
#include <node_api.h>

#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "pfhip.h"

namespace {

napi_value undefined_value(napi_env env) {
  napi_value u;
  napi_get_undefined(env, &u);
  return u;
}

napi_value throw_error(napi_env env, const std::string& msg) {
  napi_throw_error(env, nullptr, msg.c_str());
  return nullptr;
}

// Arguments of one call; `ok` turns false (with a JS exception pending) on
// the first argument of the wrong type.
struct Args {
  napi_env env;
  const char* fn;
  std::vector<napi_value> v;
  bool ok = true;

  Args(napi_env e, napi_callback_info info, size_t want, const char* name) : env(e), fn(name), v(want) {
    size_t argc = want;
    if (napi_get_cb_info(env, info, &argc, v.data(), nullptr, nullptr) != napi_ok) {
      fail("could not read arguments");
      return;
    }
    v.resize(argc);
  }
  size_t count() const { return v.size(); }
  void fail(const std::string& what) {
    if (ok) throw_error(env, std::string(fn) + ": " + what);
    ok = false;
  }
  bool require(size_t n) {
    if (v.size() < n) fail("requires " + std::to_string(n) + " arguments");
    return ok;
  }
  bool is_nullish(size_t i) {
    if (i >= v.size()) return true;
    napi_valuetype t;
    napi_typeof(env, v[i], &t);
    return t == napi_null || t == napi_undefined;
  }
  uint64_t handle(size_t i, const char* what) {
    if (!ok) return 0;
    uint64_t raw = 0;
    bool lossless = false;
    if (napi_get_value_bigint_uint64(env, v[i], &raw, &lossless) != napi_ok || raw == 0) {
      fail(std::string("argument ") + std::to_string(i) + " must be a non-null BigInt " + what + " handle");
      return 0;
    }
    return raw;
  }
  uint32_t u32(size_t i, const char* what) {
    if (!ok) return 0;
    uint32_t x = 0;
    if (napi_get_value_uint32(env, v[i], &x) != napi_ok) fail(std::string("argument ") + std::to_string(i) + " (" +
                                                              what + ") must be a non-negative integer");
    return x;
  }
  double number(size_t i, const char* what) {
    if (!ok) return 0;
    double x = 0;
    if (napi_get_value_double(env, v[i], &x) != napi_ok) fail(std::string(what) + " must be a number");
    return x;
  }
  std::string str(size_t i, const char* what) {
    if (!ok) return {};
    size_t n = 0;
    if (napi_get_value_string_utf8(env, v[i], nullptr, 0, &n) != napi_ok) {
      fail(std::string("argument ") + std::to_string(i) + " (" + what + ") must be a string");
      return {};
    }
    std::string s(n, '\0');
    napi_get_value_string_utf8(env, v[i], &s[0], n + 1, &n);
    return s;
  }
  // Bytes of a typed array of the given element type (napi_uint8_array etc.).
  void* typed(size_t i, napi_typedarray_type want, size_t* count, const char* what) {
    if (!ok) return nullptr;
    bool is = false;
    napi_is_typedarray(env, v[i], &is);
    napi_typedarray_type t;
    size_t len = 0, off = 0;
    void* data = nullptr;
    napi_value ab;
    if (!is || napi_get_typedarray_info(env, v[i], &t, &len, &data, &ab, &off) != napi_ok || t != want) {
      fail(std::string("argument ") + std::to_string(i) + " must be a " + what);
      return nullptr;
    }
    *count = len;
    return data;
  }
  // BigInt[] of buffer handles (at most 16).
  std::vector<pfhip_buffer*> bindings(size_t i) {
    std::vector<pfhip_buffer*> out;
    if (!ok) return out;
    bool is = false;
    uint32_t n = 0;
    if (napi_is_array(env, v[i], &is) != napi_ok || !is || napi_get_array_length(env, v[i], &n) != napi_ok) {
      fail("bindings must be an Array of BigInt buffer handles");
      return out;
    }
    if (n > 16) {
      fail("too many bindings (max 16)");
      return out;
    }
    for (uint32_t k = 0; k < n; ++k) {
      napi_value item;
      uint64_t raw = 0;
      bool lossless = false;
      if (napi_get_element(env, v[i], k, &item) != napi_ok ||
          napi_get_value_bigint_uint64(env, item, &raw, &lossless) != napi_ok || raw == 0) {
        fail("bindings[" + std::to_string(k) + "] must be a non-null BigInt buffer handle");
        return {};
      }
      out.push_back(reinterpret_cast<pfhip_buffer*>(static_cast<uintptr_t>(raw)));
    }
    return out;
  }
  // [gx, gy, gz] (accepted for interface parity; the HIP kernels derive their grids)
  void grid(size_t i, uint32_t g[3]) {
    if (!ok) return;
    bool is = false;
    uint32_t n = 0;
    if (napi_is_array(env, v[i], &is) != napi_ok || !is || napi_get_array_length(env, v[i], &n) != napi_ok || n != 3) {
      fail("grid must be [gx, gy, gz]");
      return;
    }
    for (uint32_t k = 0; k < 3; ++k) {
      napi_value item;
      napi_get_element(env, v[i], k, &item);
      if (napi_get_value_uint32(env, item, &g[k]) != napi_ok) {
        fail("grid entries must be non-negative integers");
        return;
      }
    }
  }
};

napi_value make_handle(napi_env env, const void* p) {
  napi_value out;
  if (napi_create_bigint_uint64(env, static_cast<uint64_t>(reinterpret_cast<uintptr_t>(p)), &out) != napi_ok)
    return throw_error(env, "napi: could not create a BigInt handle");
  return out;
}

napi_value make_string(napi_env env, const std::string& s) {
  napi_value out;
  napi_create_string_utf8(env, s.data(), s.size(), &out);
  return out;
}

// A new typed array of n elements of `bytes_per` bytes; *data receives its storage.
napi_value new_typed(napi_env env, napi_typedarray_type t, size_t n, size_t bytes_per, void** data) {
  napi_value ab, out;
  if (napi_create_arraybuffer(env, n * bytes_per, data, &ab) != napi_ok ||
      napi_create_typedarray(env, t, n, ab, 0, &out) != napi_ok)
    return throw_error(env, "napi: could not allocate the output array");
  return out;
}

template <class T>
T* as(uint64_t raw) {
  return reinterpret_cast<T*>(static_cast<uintptr_t>(raw));
}

// ---------------------------------------------------------------- NativeApi verbs

napi_value CreateBackend(napi_env env, napi_callback_info info) {
  Args a(env, info, 1, "hipCreateBackend");
  if (!a.ok) return nullptr;
  const uint32_t dev = a.is_nullish(0) ? 0 : a.u32(0, "device");
  if (!a.ok) return nullptr;
  char err[PFHIP_ERR_CAP] = {0};
  pfhip_backend* b = pfhip_create_backend(static_cast<int>(dev), err, sizeof err);
  if (!b) return throw_error(env, std::string("hip: createBackend failed: ") + err);
  return make_handle(env, b);
}

napi_value DestroyBackend(napi_env env, napi_callback_info info) {
  Args a(env, info, 1, "hipDestroyBackend");
  if (!a.require(1)) return nullptr;
  uint64_t raw = 0;
  bool lossless = false;
  if (napi_get_value_bigint_uint64(env, a.v[0], &raw, &lossless) != napi_ok)
    return throw_error(env, "hipDestroyBackend: argument 0 must be a BigInt backend handle");
  if (raw) pfhip_destroy_backend(as<pfhip_backend>(raw));
  return undefined_value(env);
}

napi_value DeviceName(napi_env env, napi_callback_info info) {
  Args a(env, info, 1, "hipDeviceName");
  if (!a.require(1)) return nullptr;
  const uint64_t h = a.handle(0, "backend");
  if (!a.ok) return nullptr;
  char name[256] = {0};
  if (pfhip_device_name(as<pfhip_backend>(h), name, sizeof name) != 0)
    return throw_error(env, "hipDeviceName: no device name");
  return make_string(env, name);
}

napi_value CreateBuffer(napi_env env, napi_callback_info info) {
  Args a(env, info, 2, "hipCreateBuffer");
  if (!a.require(2)) return nullptr;
  const uint64_t h = a.handle(0, "backend");
  size_t n = 0;
  void* data = a.typed(1, napi_uint8_array, &n, "Uint8Array (bytes)");
  if (!a.ok) return nullptr;
  char err[PFHIP_ERR_CAP] = {0};
  pfhip_buffer* buf = pfhip_create_buffer(as<pfhip_backend>(h), data, n, err, sizeof err);
  if (!buf) return throw_error(env, std::string("hip: createBuffer failed: ") + err);
  return make_handle(env, buf);
}

napi_value CreateEmptyBuffer(napi_env env, napi_callback_info info) {
  Args a(env, info, 2, "hipCreateEmptyBuffer");
  if (!a.require(2)) return nullptr;
  const uint64_t h = a.handle(0, "backend");
  const double n = a.number(1, "byteLen");
  if (!a.ok) return nullptr;
  if (!(n >= 0) || n > 9.0e15) return throw_error(env, "hipCreateEmptyBuffer: byteLen out of range");
  char err[PFHIP_ERR_CAP] = {0};
  pfhip_buffer* buf = pfhip_create_empty_buffer(as<pfhip_backend>(h), static_cast<size_t>(n), err, sizeof err);
  if (!buf) return throw_error(env, std::string("hip: createEmptyBuffer failed: ") + err);
  return make_handle(env, buf);
}

napi_value ReleaseBuffer(napi_env env, napi_callback_info info) {
  Args a(env, info, 2, "hipReleaseBuffer");
  if (!a.require(2)) return nullptr;
  const uint64_t h = a.handle(0, "backend");
  const uint64_t buf = a.handle(1, "buffer");
  if (!a.ok) return nullptr;
  pfhip_release_buffer(as<pfhip_backend>(h), as<pfhip_buffer>(buf));
  return undefined_value(env);
}

napi_value WriteBuffer(napi_env env, napi_callback_info info) {
  Args a(env, info, 4, "hipWriteBuffer");
  if (!a.require(4)) return nullptr;
  const uint64_t h = a.handle(0, "backend");
  const uint64_t buf = a.handle(1, "buffer");
  const double off = a.number(2, "offset");
  size_t n = 0;
  void* data = a.typed(3, napi_uint8_array, &n, "Uint8Array (bytes)");
  if (!a.ok) return nullptr;
  if (!(off >= 0)) return throw_error(env, "hipWriteBuffer: offset must be non-negative");
  char err[PFHIP_ERR_CAP] = {0};
  if (pfhip_write_buffer(as<pfhip_backend>(h), as<pfhip_buffer>(buf), static_cast<size_t>(off), data, n, err,
                         sizeof err) != 0)
    return throw_error(env, std::string("hip: writeBuffer failed: ") + err);
  return undefined_value(env);
}

napi_value ReadBuffer(napi_env env, napi_callback_info info) {
  Args a(env, info, 4, "hipReadBuffer");
  if (!a.require(4)) return nullptr;
  const uint64_t h = a.handle(0, "backend");
  const uint64_t buf = a.handle(1, "buffer");
  const double off = a.number(2, "offset"), n = a.number(3, "byteLen");
  if (!a.ok) return nullptr;
  if (!(off >= 0) || !(n >= 0)) return throw_error(env, "hipReadBuffer: offset and byteLen must be non-negative");
  void* dst = nullptr;
  napi_value out = new_typed(env, napi_uint8_array, static_cast<size_t>(n), 1, &dst);
  if (!out) return nullptr;
  char err[PFHIP_ERR_CAP] = {0};
  if (pfhip_read_buffer(as<pfhip_backend>(h), as<pfhip_buffer>(buf), static_cast<size_t>(off), dst,
                        static_cast<size_t>(n), err, sizeof err) != 0)
    return throw_error(env, std::string("hip: readBuffer failed: ") + err);
  return out;
}

napi_value DispatchOneShot(napi_env env, napi_callback_info info) {
  Args a(env, info, 5, "hipDispatchOneShot");
  if (!a.require(5)) return nullptr;
  const uint64_t h = a.handle(0, "backend");
  const std::string name = a.str(1, "kernel name");
  std::vector<pfhip_buffer*> bs = a.bindings(2);
  size_t plen = 0;
  void* push = a.typed(3, napi_uint8_array, &plen, "Uint8Array (pushData)");
  uint32_t grid[3] = {1, 1, 1};
  a.grid(4, grid);
  if (!a.ok) return nullptr;
  char err[PFHIP_ERR_CAP] = {0};
  if (pfhip_dispatch_one_shot(as<pfhip_backend>(h), name.c_str(), bs.data(), static_cast<uint32_t>(bs.size()), push,
                              plen, grid, err, sizeof err) != 0)
    return throw_error(env, std::string("hip: dispatchOneShot failed: ") + err);
  return undefined_value(env);
}

napi_value BeginEncoder(napi_env env, napi_callback_info info) {
  Args a(env, info, 1, "hipBeginEncoder");
  if (!a.require(1)) return nullptr;
  const uint64_t h = a.handle(0, "backend");
  if (!a.ok) return nullptr;
  char err[PFHIP_ERR_CAP] = {0};
  pfhip_encoder* e = pfhip_begin_encoder(as<pfhip_backend>(h), err, sizeof err);
  if (!e) return throw_error(env, std::string("hip: beginEncoder failed: ") + err);
  return make_handle(env, e);
}

napi_value EnqueueDispatch(napi_env env, napi_callback_info info) {
  Args a(env, info, 5, "hipEnqueueDispatch");
  if (!a.require(5)) return nullptr;
  const uint64_t e = a.handle(0, "encoder");
  const std::string name = a.str(1, "kernel name");
  std::vector<pfhip_buffer*> bs = a.bindings(2);
  size_t plen = 0;
  void* push = a.typed(3, napi_uint8_array, &plen, "Uint8Array (pushData)");
  uint32_t grid[3] = {1, 1, 1};
  a.grid(4, grid);
  if (!a.ok) return nullptr;
  char err[PFHIP_ERR_CAP] = {0};
  if (pfhip_enqueue_dispatch(as<pfhip_encoder>(e), name.c_str(), bs.data(), static_cast<uint32_t>(bs.size()), push,
                             plen, grid, err, sizeof err) != 0)
    return throw_error(env, std::string("hip: enqueueDispatch failed: ") + err);
  return undefined_value(env);
}

napi_value SubmitAndReadback(napi_env env, napi_callback_info info) {
  Args a(env, info, 4, "hipSubmitAndReadback");
  if (!a.require(4)) return nullptr;
  const uint64_t e = a.handle(0, "encoder");
  const uint64_t buf = a.handle(1, "buffer");
  const double off = a.number(2, "offset"), n = a.number(3, "byteLen");
  if (!a.ok) return nullptr;
  if (!(off >= 0) || !(n >= 0)) return throw_error(env, "hipSubmitAndReadback: offset and byteLen must be non-negative");
  void* dst = nullptr;
  napi_value out = new_typed(env, napi_uint8_array, static_cast<size_t>(n), 1, &dst);
  if (!out) return nullptr;
  char err[PFHIP_ERR_CAP] = {0};
  if (pfhip_submit_and_readback(as<pfhip_encoder>(e), as<pfhip_buffer>(buf), static_cast<size_t>(off), dst,
                                static_cast<size_t>(n), err, sizeof err) != 0)
    return throw_error(env, std::string("hip: submitAndReadback failed: ") + err);
  return out;
}

napi_value KernelNames(napi_env env, napi_callback_info) { return make_string(env, pfhip_kernel_names()); }
napi_value Version(napi_env env, napi_callback_info) { return make_string(env, pfhip_version()); }

// ---------------------------------------------------------------- whole forward

// config: {hidden, heads, kvHeads, headDim, window, dff, experts, topk, classes,
// vocab, layers, eps, ropeTheta, ropeFactor, ropeBetaFast, ropeBetaSlow,
// ropeOrigMax, ropeTruncate, precision}; missing keys take the
// privacy-filter values (native/backend.ts:392-404).
bool read_config(napi_env env, napi_value obj, pfhip_model_config* c) {
  *c = pfhip_model_config{640, 14, 2, 64, 128, 640, 128, 4, 33, 200064, 8, 1e-5f, 150000.0, 32.0, 32.0, 1.0,
                          4096, 0, PFHIP_PRECISION_FP16};
  napi_valuetype t;
  napi_typeof(env, obj, &t);
  if (t == napi_undefined || t == napi_null) return true;
  if (t != napi_object) {
    throw_error(env, "hipModelCreate: config must be an object");
    return false;
  }
  auto get = [&](const char* key, double* out) -> bool {
    bool has = false;
    napi_has_named_property(env, obj, key, &has);
    if (!has) return true;
    napi_value v;
    napi_get_named_property(env, obj, key, &v);
    if (napi_get_value_double(env, v, out) != napi_ok) {
      throw_error(env, std::string("hipModelCreate: config.") + key + " must be a number");
      return false;
    }
    return true;
  };
  struct U {
    const char* k;
    uint32_t* p;
  } us[] = {{"hidden", &c->hidden},   {"heads", &c->heads},       {"kvHeads", &c->kv_heads},
            {"headDim", &c->head_dim}, {"window", &c->window},    {"dff", &c->dff},
            {"experts", &c->experts}, {"topk", &c->topk},         {"classes", &c->classes},
            {"vocab", &c->vocab},     {"layers", &c->layers},     {"ropeOrigMax", &c->rope_orig_max},
            {"ropeTruncate", &c->rope_truncate}, {"precision", &c->precision}};
  for (auto& u : us) {
    double d = *u.p;
    if (!get(u.k, &d)) return false;
    if (!(d >= 0) || d > 4294967295.0) {
      throw_error(env, std::string("hipModelCreate: config.") + u.k + " out of range");
      return false;
    }
    *u.p = static_cast<uint32_t>(d);
  }
  double eps = c->eps;
  if (!get("eps", &eps) || !get("ropeTheta", &c->rope_theta) || !get("ropeFactor", &c->rope_factor) ||
      !get("ropeBetaFast", &c->rope_beta_fast) || !get("ropeBetaSlow", &c->rope_beta_slow))
    return false;
  c->eps = static_cast<float>(eps);
  return true;
}

napi_value ModelCreate(napi_env env, napi_callback_info info) {
  Args a(env, info, 2, "hipModelCreate");
  if (!a.require(1)) return nullptr;
  const uint64_t h = a.handle(0, "backend");
  if (!a.ok) return nullptr;
  pfhip_model_config c;
  if (!read_config(env, a.count() > 1 ? a.v[1] : nullptr, &c)) return nullptr;
  char err[PFHIP_ERR_CAP] = {0};
  pfhip_model* m = pfhip_model_create(as<pfhip_backend>(h), &c, err, sizeof err);
  if (!m) return throw_error(env, std::string("hip: modelCreate failed: ") + err);
  return make_handle(env, m);
}

napi_value ModelDestroy(napi_env env, napi_callback_info info) {
  Args a(env, info, 1, "hipModelDestroy");
  if (!a.require(1)) return nullptr;
  uint64_t raw = 0;
  bool lossless = false;
  if (napi_get_value_bigint_uint64(env, a.v[0], &raw, &lossless) != napi_ok)
    return throw_error(env, "hipModelDestroy: argument 0 must be a BigInt model handle");
  if (raw) pfhip_model_destroy(as<pfhip_model>(raw));
  return undefined_value(env);
}

napi_value ModelSetWeight(napi_env env, napi_callback_info info) {
  Args a(env, info, 3, "hipModelSetWeight");
  if (!a.require(3)) return nullptr;
  const uint64_t m = a.handle(0, "model");
  const std::string name = a.str(1, "weight name");
  size_t n = 0;
  void* data = a.typed(2, napi_uint8_array, &n, "Uint8Array (bytes)");
  if (!a.ok) return nullptr;
  char err[PFHIP_ERR_CAP] = {0};
  if (pfhip_model_set_weight(as<pfhip_model>(m), name.c_str(), data, n, err, sizeof err) != 0)
    return throw_error(env, std::string("hip: modelSetWeight failed: ") + err);
  return undefined_value(env);
}

napi_value ModelFinalize(napi_env env, napi_callback_info info) {
  Args a(env, info, 1, "hipModelFinalize");
  if (!a.require(1)) return nullptr;
  const uint64_t m = a.handle(0, "model");
  if (!a.ok) return nullptr;
  char err[PFHIP_ERR_CAP] = {0};
  if (pfhip_model_finalize(as<pfhip_model>(m), err, sizeof err) != 0)
    return throw_error(env, std::string("hip: modelFinalize failed: ") + err);
  return undefined_value(env);
}

// hipForward(m, Int32Array ids, Uint8Array|null mask, batch, seqLen) -> Float32Array [batch*seqLen*classes]
napi_value Forward(napi_env env, napi_callback_info info) {
  Args a(env, info, 6, "hipForward");
  if (!a.require(5)) return nullptr;
  const uint64_t m = a.handle(0, "model");
  size_t n_ids = 0, n_mask = 0;
  const void* ids = a.typed(1, napi_int32_array, &n_ids, "Int32Array (tokenIds)");
  const void* mask = a.is_nullish(2) ? nullptr : a.typed(2, napi_uint8_array, &n_mask, "Uint8Array (attentionMask)");
  const uint32_t batch = a.u32(3, "batch"), seq = a.u32(4, "seqLen");
  const uint32_t classes = a.count() > 5 && !a.is_nullish(5) ? a.u32(5, "numClasses") : 33u;
  if (!a.ok) return nullptr;
  if ((size_t)batch * seq != n_ids) return throw_error(env, "hipForward: tokenIds length must be batch * seqLen");
  if (mask && n_mask != n_ids)
    return throw_error(env, "hipForward: attentionMask length " + std::to_string(n_mask) +
                                " does not match tokenIds length " + std::to_string(n_ids));
  void* dst = nullptr;
  napi_value out = new_typed(env, napi_float32_array, n_ids * classes, 4, &dst);
  if (!out) return nullptr;
  char err[PFHIP_ERR_CAP] = {0};
  if (pfhip_model_forward(as<pfhip_model>(m), static_cast<const int32_t*>(ids), static_cast<const uint8_t*>(mask),
                          batch, seq, static_cast<float*>(dst), err, sizeof err) != 0)
    return throw_error(env, std::string("hip: forward failed: ") + err);
  return out;
}

// ---------------------------------------------------------------- spans (host only)

napi_value ViterbiDecode(napi_env env, napi_callback_info info) {
  Args a(env, info, 6, "hipViterbiDecode");
  if (!a.require(5)) return nullptr;
  size_t n_logits = 0, n_lens = 0, n_bias = 0;
  const void* logits = a.typed(0, napi_float32_array, &n_logits, "Float32Array (logits)");
  const uint32_t batch = a.u32(1, "batch"), stride = a.u32(2, "seqStride");
  const void* lens = a.is_nullish(3) ? nullptr : a.typed(3, napi_uint32_array, &n_lens, "Uint32Array (seqLens)");
  const void* biases = a.typed(4, napi_float32_array, &n_bias, "Float32Array (biases)");
  const uint32_t threads = a.count() > 5 && !a.is_nullish(5) ? a.u32(5, "nThreads") : 0u;
  if (!a.ok) return nullptr;
  const uint32_t classes = 33;
  if (n_logits != (size_t)batch * stride * classes)
    return throw_error(env, "hipViterbiDecode: logits length must be batch * seqStride * 33");
  if (lens && n_lens != batch) return throw_error(env, "hipViterbiDecode: seqLens length must be batch");
  if (n_bias != 6) return throw_error(env, "hipViterbiDecode: biases must hold the 6 calibration biases");
  void* dst = nullptr;
  napi_value out = new_typed(env, napi_uint8_array, (size_t)batch * stride, 1, &dst);
  if (!out) return nullptr;
  char err[PFHIP_ERR_CAP] = {0};
  if (pfhip_viterbi_decode(static_cast<const float*>(logits), batch, stride, static_cast<const uint32_t*>(lens),
                           classes, static_cast<const float*>(biases), static_cast<uint8_t*>(dst), threads, err,
                           sizeof err) != 0)
    return throw_error(env, std::string("hip: viterbiDecode failed: ") + err);
  return out;
}

napi_value Init(napi_env env, napi_value exports) {
  struct {
    const char* name;
    napi_callback cb;
  } fns[] = {{"hipCreateBackend", CreateBackend},
             {"hipDestroyBackend", DestroyBackend},
             {"hipDeviceName", DeviceName},
             {"hipCreateBuffer", CreateBuffer},
             {"hipCreateEmptyBuffer", CreateEmptyBuffer},
             {"hipReleaseBuffer", ReleaseBuffer},
             {"hipWriteBuffer", WriteBuffer},
             {"hipReadBuffer", ReadBuffer},
             {"hipDispatchOneShot", DispatchOneShot},
             {"hipBeginEncoder", BeginEncoder},
             {"hipEnqueueDispatch", EnqueueDispatch},
             {"hipSubmitAndReadback", SubmitAndReadback},
             {"hipKernelNames", KernelNames},
             {"hipVersion", Version},
             {"hipModelCreate", ModelCreate},
             {"hipModelDestroy", ModelDestroy},
             {"hipModelSetWeight", ModelSetWeight},
             {"hipModelFinalize", ModelFinalize},
             {"hipForward", Forward},
             {"hipViterbiDecode", ViterbiDecode}};
  for (auto& f : fns) {
    napi_value fn;
    if (napi_create_function(env, f.name, NAPI_AUTO_LENGTH, f.cb, nullptr, &fn) != napi_ok ||
        napi_set_named_property(env, exports, f.name, fn) != napi_ok)
      return nullptr;
  }
  return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, Init)
