// N-API addon: the Node binding of libchonk.so for the TypeScript host
// (chonklm_amd/node/llama-hip-runtime.js mirrors src/lib/llama-wgsl-runtime.ts).
//
// Every call that runs device work (engine creation, runToken, generate) is
// an N-API async work item and returns a Promise, as the reference's
// runToken / generateLlamaWgsl / loadLlamaWgslModel do; cheap queries
// (position, readLogits, reset, dispose) are synchronous. Errors reject with
// a JS Error carrying the engine's message (the reference's wording) and a
// `code` property holding the status name.
//
// The stepped generate delivers the reference's shouldStop / onToken events
// through a thread-safe function: the worker thread blocks until the JS
// callback has run and returned.
#include <node_api.h>

#include <algorithm>
#include <condition_variable>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "chonk.h"

namespace {

#define NAPI_OK(call)                                                        \
  do {                                                                       \
    if ((call) != napi_ok) {                                                 \
      napi_throw_error(env, nullptr, "N-API call failed: " #call);           \
      return nullptr;                                                        \
    }                                                                        \
  } while (0)

const char* status_name(int rc) {
  switch (rc) {
    case CHONK_EINVAL: return "EINVAL";
    case CHONK_EIO: return "EIO";
    case CHONK_EHIP: return "EHIP";
    case CHONK_ECONTEXT: return "ECONTEXT";
    case CHONK_EBUSY: return "EBUSY";
    case CHONK_ELOST: return "ELOST";
    case CHONK_ENOMEM: return "ENOMEM";
    default: return "ERROR";
  }
}

napi_value make_error(napi_env env, int rc, const std::string& msg) {
  napi_value m, code, err;
  napi_create_string_utf8(env, msg.c_str(), msg.size(), &m);
  napi_create_string_utf8(env, status_name(rc), NAPI_AUTO_LENGTH, &code);
  napi_create_error(env, code, m, &err);
  return err;
}

std::string engine_error(chonk_engine* e, int rc) {
  const char* m = e ? chonk_engine_last_error(e) : chonk_last_error();
  std::string s = (m && *m) ? m : "";
  if (s.empty()) s = std::string("libchonk call failed with ") + status_name(rc);
  return s;
}

// Engine handle: a JS external wrapping the engine pointer; destroyed by
// dispose() or by the garbage collector.
struct Handle {
  chonk_engine* e = nullptr;
};

void finalize_handle(napi_env, void* data, void*) {
  Handle* h = static_cast<Handle*>(data);
  if (h->e) chonk_engine_destroy(h->e);
  delete h;
}

Handle* get_handle(napi_env env, napi_value v) {
  void* data = nullptr;
  if (napi_get_value_external(env, v, &data) != napi_ok || !data) {
    napi_throw_type_error(env, nullptr, "expected an engine handle");
    return nullptr;
  }
  Handle* h = static_cast<Handle*>(data);
  if (!h->e) {
    napi_throw_error(env, "EINVAL", "engine was disposed");
    return nullptr;
  }
  return h;
}

bool get_prop(napi_env env, napi_value obj, const char* key, napi_value* out) {
  bool has = false;
  if (napi_has_named_property(env, obj, key, &has) != napi_ok || !has) return false;
  if (napi_get_named_property(env, obj, key, out) != napi_ok) return false;
  napi_valuetype t;
  napi_typeof(env, *out, &t);
  return t != napi_undefined && t != napi_null;
}

double num_prop(napi_env env, napi_value obj, const char* key, double dflt) {
  napi_value v;
  double d = dflt;
  if (get_prop(env, obj, key, &v) && napi_get_value_double(env, v, &d) != napi_ok) d = dflt;
  return d;
}

std::string str_prop(napi_env env, napi_value obj, const char* key) {
  napi_value v;
  if (!get_prop(env, obj, key, &v)) return "";
  size_t n = 0;
  if (napi_get_value_string_utf8(env, v, nullptr, 0, &n) != napi_ok) return "";
  std::string s(n, '\0');
  napi_get_value_string_utf8(env, v, &s[0], n + 1, &n);
  return s;
}

std::vector<int32_t> int_array(napi_env env, napi_value v) {
  std::vector<int32_t> out;
  bool is_arr = false, is_typed = false;
  napi_is_array(env, v, &is_arr);
  napi_is_typedarray(env, v, &is_typed);
  if (is_typed) {
    napi_typedarray_type t;
    size_t len = 0;
    void* data = nullptr;
    napi_get_typedarray_info(env, v, &t, &len, &data, nullptr, nullptr);
    if (t == napi_int32_array || t == napi_uint32_array) {
      out.assign((const int32_t*)data, (const int32_t*)data + len);
      return out;
    }
  }
  if (!is_arr) return out;
  uint32_t n = 0;
  napi_get_array_length(env, v, &n);
  out.resize(n);
  for (uint32_t i = 0; i < n; ++i) {
    napi_value x;
    napi_get_element(env, v, i, &x);
    double d = 0;
    napi_get_value_double(env, x, &d);
    out[i] = (int32_t)d;
  }
  return out;
}

chonk_sampling sampling_from(napi_env env, napi_value opts) {
  chonk_sampling s{};
  s.temperature = 0;
  s.top_p = 1;
  s.top_k = 0;
  s.repetition_penalty = 1;
  s.seed = 0;
  napi_valuetype t = napi_undefined;
  if (opts) napi_typeof(env, opts, &t);
  if (t != napi_object) return s;
  s.temperature = num_prop(env, opts, "temperature", 0);
  s.top_p = num_prop(env, opts, "topP", 1);
  // normalizeTopK (sampling.ts:78-81): non-finite -> 0, floor, clamp at 0
  const double k = num_prop(env, opts, "topK", 0);
  s.top_k = (k == k && k > 0 && k < 2147483647.0) ? (int32_t)k : 0;
  s.repetition_penalty = num_prop(env, opts, "repetitionPenalty", 1);
  s.seed = (uint64_t)num_prop(env, opts, "seed", 0);
  return s;
}

napi_value make_int_array(napi_env env, const std::vector<int32_t>& v) {
  napi_value arr;
  napi_create_array_with_length(env, v.size(), &arr);
  for (size_t i = 0; i < v.size(); ++i) {
    napi_value x;
    napi_create_int32(env, v[i], &x);
    napi_set_element(env, arr, (uint32_t)i, x);
  }
  return arr;
}

// ---- async work ------------------------------------------------------------------

struct Work {
  napi_async_work work = nullptr;
  napi_deferred deferred = nullptr;
  napi_ref handle_ref = nullptr;  // keeps the engine external alive while the work runs
  Handle* h = nullptr;
  int rc = CHONK_OK;
  std::string err;
  virtual ~Work() = default;
  virtual void execute() = 0;
  virtual napi_value result(napi_env env) = 0;
};

void work_execute(napi_env, void* data) {
  Work* w = static_cast<Work*>(data);
  w->execute();
}

void work_complete(napi_env env, napi_status, void* data) {
  Work* w = static_cast<Work*>(data);
  if (w->rc == CHONK_OK) {
    napi_resolve_deferred(env, w->deferred, w->result(env));
  } else {
    napi_reject_deferred(env, w->deferred, make_error(env, w->rc, w->err));
  }
  if (w->handle_ref) napi_delete_reference(env, w->handle_ref);
  napi_delete_async_work(env, w->work);
  delete w;
}

napi_value queue(napi_env env, Work* w, const char* name, napi_value handle_value) {
  napi_value promise, res_name;
  if (napi_create_promise(env, &w->deferred, &promise) != napi_ok) {
    delete w;
    napi_throw_error(env, nullptr, "could not create a promise");
    return nullptr;
  }
  if (handle_value) napi_create_reference(env, handle_value, 1, &w->handle_ref);
  napi_create_string_utf8(env, name, NAPI_AUTO_LENGTH, &res_name);
  napi_create_async_work(env, nullptr, res_name, work_execute, work_complete, w, &w->work);
  napi_queue_async_work(env, w->work);
  return promise;
}

// createEngine(def, path) -> Promise<handle>
struct CreateWork : Work {
  std::string id, path;
  std::vector<int32_t> eos;
  chonk_model_def def{};
  chonk_engine* out = nullptr;
  void execute() override {
    def.id = id.c_str();
    def.eos_ids = eos.data();
    def.n_eos = (int32_t)eos.size();
    rc = chonk_engine_create(&def, path.c_str(), &out);
    if (rc != CHONK_OK) err = engine_error(nullptr, rc);
  }
  napi_value result(napi_env env) override {
    Handle* h = new Handle();
    h->e = out;
    napi_value ext;
    napi_create_external(env, h, finalize_handle, nullptr, &ext);
    return ext;
  }
};

napi_value CreateEngine(napi_env env, napi_callback_info info) {
  size_t argc = 2;
  napi_value argv[2];
  NAPI_OK(napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr));
  if (argc < 2) {
    napi_throw_type_error(env, nullptr, "createEngine(def, path)");
    return nullptr;
  }
  CreateWork* w = new CreateWork();
  w->id = str_prop(env, argv[0], "id");
  w->def.vocab = (int32_t)num_prop(env, argv[0], "vocab", 0);
  w->def.layers = (int32_t)num_prop(env, argv[0], "layers", 0);
  w->def.max_context = (int32_t)num_prop(env, argv[0], "maxContext", 0);
  w->def.default_repetition_penalty = (float)num_prop(env, argv[0], "defaultRepetitionPenalty", 0);
  w->def.kv_dtype = str_prop(env, argv[0], "kvDtype") == "float32" ? CHONK_KV_F32 : CHONK_KV_F16;
  w->def.device = (int32_t)num_prop(env, argv[0], "device", 0);
  napi_value eos;
  if (get_prop(env, argv[0], "eosIds", &eos)) w->eos = int_array(env, eos);
  size_t n = 0;
  napi_get_value_string_utf8(env, argv[1], nullptr, 0, &n);
  w->path.assign(n, '\0');
  napi_get_value_string_utf8(env, argv[1], &w->path[0], n + 1, &n);
  return queue(env, w, "chonk.createEngine", nullptr);
}

// runToken(handle, token, needLogits, opts, penalized, seen) -> Promise<number>
struct RunWork : Work {
  int32_t token = 0, need = 0, out = 0;
  chonk_sampling s{};
  std::vector<int32_t> pen, seen;
  void execute() override {
    rc = chonk_engine_run_token(h->e, token, need, &s, pen.data(), pen.size(), seen.data(), seen.size(), &out);
    if (rc != CHONK_OK) err = engine_error(h->e, rc);
  }
  napi_value result(napi_env env) override {
    napi_value v;
    napi_create_int32(env, out, &v);
    return v;
  }
};

napi_value RunToken(napi_env env, napi_callback_info info) {
  size_t argc = 6;
  napi_value argv[6];
  NAPI_OK(napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr));
  Handle* h = argc > 0 ? get_handle(env, argv[0]) : nullptr;
  if (!h) return nullptr;
  RunWork* w = new RunWork();
  w->h = h;
  double d = 0;
  if (argc > 1) napi_get_value_double(env, argv[1], &d);
  w->token = (int32_t)d;
  bool need = false;
  if (argc > 2) napi_get_value_bool(env, argv[2], &need);
  w->need = need ? 1 : 0;
  w->s = sampling_from(env, argc > 3 ? argv[3] : nullptr);
  if (argc > 4) w->pen = int_array(env, argv[4]);
  if (argc > 5) w->seen = int_array(env, argv[5]);
  return queue(env, w, "chonk.runToken", argv[0]);
}

// generate(handle, promptIds, maxNewTokens, opts, callback?) -> Promise<{ids, stats}>
struct StepBridge {
  napi_threadsafe_function tsfn = nullptr;
  std::mutex mu;
  std::condition_variable cv;
  bool done = false;
  int32_t event = 0, token = 0, result = 0;
};

void call_js(napi_env env, napi_value js_cb, void*, void* data) {
  StepBridge* b = static_cast<StepBridge*>(data);
  int32_t result = 0;
  if (env && js_cb) {
    napi_value argv[2], ret, undef;
    napi_create_int32(env, b->event, &argv[0]);
    napi_create_int32(env, b->token, &argv[1]);
    napi_get_undefined(env, &undef);
    if (napi_call_function(env, undef, js_cb, 2, argv, &ret) == napi_ok) {
      bool bv = false;
      napi_valuetype t;
      napi_typeof(env, ret, &t);
      if (t == napi_boolean) {
        napi_get_value_bool(env, ret, &bv);
        result = bv ? 1 : 0;
      } else if (t == napi_number) {
        double d = 0;
        napi_get_value_double(env, ret, &d);
        result = d != 0 ? 1 : 0;
      }
    } else {
      // an exception in the callback stops generation; clear it so the promise can settle
      napi_value exc;
      napi_get_and_clear_last_exception(env, &exc);
      result = 1;
    }
  } else {
    result = 1;
  }
  std::lock_guard<std::mutex> lk(b->mu);
  b->result = result;
  b->done = true;
  b->cv.notify_one();
}

int32_t bridge_callback(void* user, int32_t event, int32_t token) {
  StepBridge* b = static_cast<StepBridge*>(user);
  std::unique_lock<std::mutex> lk(b->mu);
  b->done = false;
  b->event = event;
  b->token = token;
  lk.unlock();
  if (napi_call_threadsafe_function(b->tsfn, b, napi_tsfn_blocking) != napi_ok) return 1;
  lk.lock();
  b->cv.wait(lk, [b] { return b->done; });
  return b->result;
}

struct GenWork : Work {
  std::vector<int32_t> prompt, out;
  int32_t max_new = 0;
  chonk_sampling s{};
  chonk_gen_stats stats{};
  StepBridge* bridge = nullptr;
  ~GenWork() override { delete bridge; }
  void execute() override {
    const size_t cap = (size_t)(max_new >= 0 ? std::max(max_new, 1) : 128);
    out.assign(cap, 0);
    size_t n = 0;
    if (bridge) {
      rc = chonk_engine_generate_stepped(h->e, prompt.data(), prompt.size(), max_new, &s, bridge_callback, bridge,
                                         out.data(), cap, &n, &stats);
      napi_release_threadsafe_function(bridge->tsfn, napi_tsfn_release);
    } else {
      rc = chonk_engine_generate(h->e, prompt.data(), prompt.size(), max_new, &s, out.data(), cap, &n, &stats);
    }
    if (rc != CHONK_OK) err = engine_error(h->e, rc);
    out.resize(std::min(n, cap));
  }
  napi_value result(napi_env env) override {
    napi_value obj, v;
    napi_create_object(env, &obj);
    napi_set_named_property(env, obj, "ids", make_int_array(env, out));
    napi_create_double(env, stats.tokens_per_sec, &v);
    napi_set_named_property(env, obj, "tokensPerSec", v);
    napi_create_double(env, stats.prefill_ms, &v);
    napi_set_named_property(env, obj, "prefillMs", v);
    napi_create_double(env, stats.decode_ms, &v);
    napi_set_named_property(env, obj, "decodeMs", v);
    return obj;
  }
};

napi_value Generate(napi_env env, napi_callback_info info) {
  size_t argc = 5;
  napi_value argv[5];
  NAPI_OK(napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr));
  Handle* h = argc > 0 ? get_handle(env, argv[0]) : nullptr;
  if (!h) return nullptr;
  GenWork* w = new GenWork();
  w->h = h;
  if (argc > 1) w->prompt = int_array(env, argv[1]);
  double d = 0;
  if (argc > 2) napi_get_value_double(env, argv[2], &d);
  w->max_new = (int32_t)d;
  w->s = sampling_from(env, argc > 3 ? argv[3] : nullptr);
  napi_valuetype t = napi_undefined;
  if (argc > 4) napi_typeof(env, argv[4], &t);
  if (t == napi_function) {
    w->bridge = new StepBridge();
    napi_value name;
    napi_create_string_utf8(env, "chonk.generate.callback", NAPI_AUTO_LENGTH, &name);
    if (napi_create_threadsafe_function(env, argv[4], nullptr, name, 0, 1, nullptr, nullptr, nullptr, call_js,
                                        &w->bridge->tsfn) != napi_ok) {
      delete w;
      napi_throw_error(env, nullptr, "could not create the token callback");
      return nullptr;
    }
  }
  return queue(env, w, "chonk.generate", argv[0]);
}

// ---- synchronous calls -------------------------------------------------------------

napi_value throw_rc(napi_env env, chonk_engine* e, int rc) {
  napi_throw(env, make_error(env, rc, engine_error(e, rc)));
  return nullptr;
}

Handle* handle_arg(napi_env env, napi_callback_info info, size_t want, napi_value* argv) {
  size_t argc = want;
  if (napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr) != napi_ok || argc < 1) {
    napi_throw_type_error(env, nullptr, "missing engine handle");
    return nullptr;
  }
  return get_handle(env, argv[0]);
}

napi_value Position(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  Handle* h = handle_arg(env, info, 1, argv);
  if (!h) return nullptr;
  int32_t p = 0;
  const int rc = chonk_engine_position(h->e, &p);
  if (rc != CHONK_OK) return throw_rc(env, h->e, rc);
  napi_value v;
  napi_create_int32(env, p, &v);
  return v;
}

napi_value Reset(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  Handle* h = handle_arg(env, info, 1, argv);
  if (!h) return nullptr;
  const int rc = chonk_engine_reset(h->e);
  if (rc != CHONK_OK) return throw_rc(env, h->e, rc);
  return nullptr;
}

napi_value ResetConversation(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  Handle* h = handle_arg(env, info, 1, argv);
  if (!h) return nullptr;
  const int rc = chonk_engine_reset_conversation(h->e);
  if (rc != CHONK_OK) return throw_rc(env, h->e, rc);
  return nullptr;
}

// conversation(handle) -> {cachedTokenIds: number[], cachedNextId: number | null}
napi_value Conversation(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  Handle* h = handle_arg(env, info, 1, argv);
  if (!h) return nullptr;
  size_t n = 0;
  int32_t next = -1;
  int rc = chonk_engine_conversation(h->e, nullptr, 0, &n, &next);
  if (rc != CHONK_OK) return throw_rc(env, h->e, rc);
  std::vector<int32_t> ids(n);
  rc = chonk_engine_conversation(h->e, ids.data(), n, &n, &next);
  if (rc != CHONK_OK) return throw_rc(env, h->e, rc);
  napi_value obj, nx;
  napi_create_object(env, &obj);
  napi_set_named_property(env, obj, "cachedTokenIds", make_int_array(env, ids));
  if (next < 0) {
    napi_get_null(env, &nx);
  } else {
    napi_create_int32(env, next, &nx);
  }
  napi_set_named_property(env, obj, "cachedNextId", nx);
  return obj;
}

napi_value ReadLogits(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  Handle* h = handle_arg(env, info, 1, argv);
  if (!h) return nullptr;
  chonk_engine_info ei{};
  int rc = chonk_engine_info_get(h->e, &ei);
  if (rc != CHONK_OK) return throw_rc(env, h->e, rc);
  napi_value ab, arr;
  void* data = nullptr;
  NAPI_OK(napi_create_arraybuffer(env, (size_t)ei.vocab * 4, &data, &ab));
  rc = chonk_engine_read_logits(h->e, (float*)data, (size_t)ei.vocab);
  if (rc != CHONK_OK) return throw_rc(env, h->e, rc);
  NAPI_OK(napi_create_typedarray(env, napi_float32_array, (size_t)ei.vocab, ab, 0, &arr));
  return arr;
}

napi_value Info(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  Handle* h = handle_arg(env, info, 1, argv);
  if (!h) return nullptr;
  chonk_engine_info ei{};
  const int rc = chonk_engine_info_get(h->e, &ei);
  if (rc != CHONK_OK) return throw_rc(env, h->e, rc);
  napi_value obj, v;
  napi_create_object(env, &obj);
  const struct {
    const char* k;
    double v;
  } f[] = {{"hidden", (double)ei.hidden},       {"ffn", (double)ei.ffn},
           {"vocab", (double)ei.vocab},         {"layers", (double)ei.layers},
           {"heads", (double)ei.heads},         {"kvHeads", (double)ei.kv_heads},
           {"headDim", (double)ei.head_dim},    {"context", (double)ei.context},
           {"weightBytesPerToken", (double)ei.weight_bytes_per_token},
           {"deviceBytes", (double)ei.device_bytes}, {"kernelsPerStep", (double)ei.kernels_per_step},
           {"noallocPrefillRows", (double)ei.noalloc_prefill_rows},
           {"architecture", (double)ei.architecture}};
  for (const auto& x : f) {
    napi_create_double(env, x.v, &v);
    napi_set_named_property(env, obj, x.k, v);
  }
  return obj;
}

napi_value Dispose(napi_env env, napi_callback_info info) {
  size_t argc = 1;
  napi_value argv[1];
  NAPI_OK(napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr));
  void* data = nullptr;
  if (argc < 1 || napi_get_value_external(env, argv[0], &data) != napi_ok || !data) return nullptr;
  Handle* h = static_cast<Handle*>(data);
  if (h->e) {
    const int rc = chonk_engine_destroy(h->e);
    if (rc != CHONK_OK) return throw_rc(env, h->e, rc);
    h->e = nullptr;
  }
  return nullptr;
}

napi_value Init(napi_env env, napi_value exports) {
  const napi_property_descriptor props[] = {
      {"createEngine", nullptr, CreateEngine, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"runToken", nullptr, RunToken, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"generate", nullptr, Generate, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"position", nullptr, Position, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"reset", nullptr, Reset, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"resetConversation", nullptr, ResetConversation, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"conversation", nullptr, Conversation, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"readLogits", nullptr, ReadLogits, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"info", nullptr, Info, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"dispose", nullptr, Dispose, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
  };
  napi_define_properties(env, exports, sizeof(props) / sizeof(props[0]), props);
  return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, Init)
