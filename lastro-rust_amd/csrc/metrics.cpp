// Runtime metrics publisher: the JSON snapshot the reference runtime publishes for its monitor
// (rust/moe-monitor/src/snapshot.rs), written by the runtime's own code here. Field names, their order and the
// state encoding ({"kind": "idle" | "reading" | "generating" | "queued" | "error", ...}) follow the reference's serde
// layout (snapshot.rs:18-139), so that the same reader accepts either runtime's file.
#include <errno.h>
#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <sys/types.h>
#include <unistd.h>

#include <chrono>
#include <deque>
#include <map>
#include <mutex>
#include <string>

#include "../../include/moert.h"

namespace moert {
int set_error(int code, const char* fmt, ...);
}
using moert::set_error;

namespace {

constexpr uint32_t kSchema = 1;  // SCHEMA (snapshot.rs:14)
constexpr size_t kMaxRequests = 32;
constexpr size_t kMaxEvents = 64;  // the reference keeps the last 64 events (rust/moe-rt/src/bin/m2a-cache.rs:419)

uint64_t now_ms() {
  return (uint64_t)std::chrono::duration_cast<std::chrono::milliseconds>(
             std::chrono::system_clock::now().time_since_epoch())
      .count();
}

// default_path (snapshot.rs:146-156): $XDG_RUNTIME_DIR/moe-rt/metrics.json, else /tmp/moe-rt-<uid>/metrics.json
// with the uid that owns /proc/self
std::string default_path() {
  const char* x = getenv("XDG_RUNTIME_DIR");
  if (x && *x) return std::string(x) + "/moe-rt/metrics.json";
  struct stat st;
  const unsigned uid = stat("/proc/self", &st) == 0 ? (unsigned)st.st_uid : 0u;
  return "/tmp/moe-rt-" + std::to_string(uid) + "/metrics.json";
}

// mkdir -p of the directory part of `path`
bool make_parent_dirs(const std::string& path, std::string* err) {
  const size_t slash = path.rfind('/');
  if (slash == std::string::npos || slash == 0) return true;
  const std::string dir = path.substr(0, slash);
  for (size_t i = 1; i <= dir.size(); i++) {
    if (i < dir.size() && dir[i] != '/') continue;
    const std::string part = dir.substr(0, i);
    if (mkdir(part.c_str(), 0700) == 0) continue;
    struct stat st;
    if (errno != EEXIST || stat(part.c_str(), &st) != 0 || !S_ISDIR(st.st_mode)) {
      *err = part + ": " + (errno == EEXIST ? "not a directory" : strerror(errno));
      return false;
    }
  }
  return true;
}

// JSON string: escapes quote, backslash and control characters; bytes that are not valid UTF-8 become U+FFFD
void put_str(std::string& o, const std::string& s) {
  o += '"';
  const unsigned char* p = (const unsigned char*)s.data();
  const size_t n = s.size();
  for (size_t i = 0; i < n;) {
    const unsigned c = p[i];
    if (c < 0x80) {
      switch (c) {
        case '"': o += "\\\""; break;
        case '\\': o += "\\\\"; break;
        case '\n': o += "\\n"; break;
        case '\r': o += "\\r"; break;
        case '\t': o += "\\t"; break;
        case '\b': o += "\\b"; break;
        case '\f': o += "\\f"; break;
        default:
          if (c < 0x20) {
            char b[8];
            snprintf(b, sizeof b, "\\u%04x", c);
            o += b;
          } else {
            o += (char)c;
          }
      }
      i++;
      continue;
    }
    // a multi-byte sequence: its length from the lead byte, continuation bytes 10xxxxxx, no overlong forms,
    // no surrogates, at most U+10FFFF
    int len = 0;
    unsigned cp = 0;
    if (c >= 0xC2 && c <= 0xDF) {
      len = 2;
      cp = c & 0x1F;
    } else if (c >= 0xE0 && c <= 0xEF) {
      len = 3;
      cp = c & 0x0F;
    } else if (c >= 0xF0 && c <= 0xF4) {
      len = 4;
      cp = c & 0x07;
    }
    bool ok = len > 0 && i + len <= n;
    for (int k = 1; ok && k < len; k++) {
      ok = (p[i + k] & 0xC0) == 0x80;
      cp = (cp << 6) | (p[i + k] & 0x3F);
    }
    if (ok) ok = !(len == 3 && (cp < 0x800 || (cp >= 0xD800 && cp <= 0xDFFF))) && !(len == 4 && (cp < 0x10000 || cp > 0x10FFFF));
    if (ok) {
      o.append((const char*)p + i, len);
      i += len;
    } else {
      o += "\xEF\xBF\xBD";
      i++;
    }
  }
  o += '"';
}

// JSON number of an f64: the shortest decimal that reads back as the same double, with ".0" on integral values (as
// serde_json writes f64); NaN and infinities are null (serde_json's encoding of non-finite floats)
void put_f64(std::string& o, double v) {
  if (v != v || v - v != 0.0) {
    o += "null";
    return;
  }
  char b[40];
  for (int prec = 1; prec <= 17; prec++) {
    snprintf(b, sizeof b, "%.*g", prec, v);
    if (strtod(b, nullptr) == v) break;
  }
  o += b;
  if (!strpbrk(b, ".eEn")) o += ".0";
}

void put_u64(std::string& o, uint64_t v) { o += std::to_string(v); }

struct Request {
  uint64_t started_ms, prompt_tokens, reused_tokens, output_tokens, duration_ms;
  double prefill_tok_s, decode_tok_s;
  std::string status;
};

struct Event {
  uint64_t ts_ms;
  std::string level, message;
};

}  // namespace

struct moert_metrics {
  std::mutex mu;
  std::string path, tmp;
  uint64_t started_ms = 0;
  uint32_t pid = 0;
  std::string name;
  uint32_t layers = 0, experts = 0, experts_per_tok = 0;
  int state = MOERT_STATE_IDLE;
  uint64_t sa = 0, sb = 0;
  std::string message;
  moert_metrics_speed speed{};
  uint64_t ctx_used = 0, ctx_max = 0;
  moert_metrics_cache cache{};
  moert_metrics_window window{};
  std::deque<Request> requests;  // most recent first
  std::map<std::string, std::string> settings;
  std::deque<Event> events;  // oldest first

  std::string json(uint64_t ts) const {
    std::string o;
    o.reserve(2048);
    o += "{\"schema\":";
    put_u64(o, kSchema);
    o += ",\"ts_ms\":";
    put_u64(o, ts);
    o += ",\"pid\":";
    put_u64(o, pid);
    o += ",\"started_ms\":";
    put_u64(o, started_ms);
    o += ",\"model\":{\"name\":";
    put_str(o, name);
    o += ",\"layers\":";
    put_u64(o, layers);
    o += ",\"experts\":";
    put_u64(o, experts);
    o += ",\"experts_per_tok\":";
    put_u64(o, experts_per_tok);
    o += "},\"state\":{\"kind\":";
    switch (state) {
      case MOERT_STATE_READING:
        o += "\"reading\",\"done\":";
        put_u64(o, sa);
        o += ",\"total\":";
        put_u64(o, sb);
        break;
      case MOERT_STATE_GENERATING:
        o += "\"generating\",\"tokens\":";
        put_u64(o, sa);
        o += ",\"max_tokens\":";
        put_u64(o, sb);
        break;
      case MOERT_STATE_QUEUED:
        o += "\"queued\",\"waiting\":";
        put_u64(o, sa);
        break;
      case MOERT_STATE_ERROR:
        o += "\"error\",\"message\":";
        put_str(o, message);
        break;
      default:
        o += "\"idle\"";
    }
    o += "},\"speed\":{\"decode_now\":";
    put_f64(o, speed.decode_now);
    o += ",\"decode_last\":";
    put_f64(o, speed.decode_last);
    o += ",\"prefill_now\":";
    put_f64(o, speed.prefill_now);
    o += ",\"prefill_request\":";
    put_f64(o, speed.prefill_request);
    o += "},\"context\":{\"used\":";
    put_u64(o, ctx_used);
    o += ",\"max\":";
    put_u64(o, ctx_max);
    o += "},\"cache\":{\"slots_total\":";
    put_u64(o, cache.slots_total);
    o += ",\"slots_resident\":";
    put_u64(o, cache.slots_resident);
    o += ",\"slots_loading\":";
    put_u64(o, cache.slots_loading);
    o += ",\"hit_frac\":";
    put_f64(o, cache.hit_frac);
    o += ",\"copy_frac\":";
    put_f64(o, cache.copy_frac);
    o += ",\"cpu_frac\":";
    put_f64(o, cache.cpu_frac);
    o += ",\"copies_inflight\":";
    put_u64(o, cache.copies_inflight);
    o += ",\"h2d_gbs\":";
    put_f64(o, cache.h2d_gbs);
    o += ",\"total_hits\":";
    put_u64(o, cache.total_hits);
    o += ",\"total_copies\":";
    put_u64(o, cache.total_copies);
    o += ",\"total_cpu\":";
    put_u64(o, cache.total_cpu);
    o += "},\"window\":{\"exposure_frac\":";
    put_f64(o, window.exposure_frac);
    o += ",\"gpu_wait_frac\":";
    put_f64(o, window.gpu_wait_frac);
    o += ",\"ms_per_token\":";
    put_f64(o, window.ms_per_token);
    o += "},\"requests\":[";
    for (size_t i = 0; i < requests.size(); i++) {
      const Request& r = requests[i];
      o += i ? ",{\"started_ms\":" : "{\"started_ms\":";
      put_u64(o, r.started_ms);
      o += ",\"prompt_tokens\":";
      put_u64(o, r.prompt_tokens);
      o += ",\"reused_tokens\":";
      put_u64(o, r.reused_tokens);
      o += ",\"output_tokens\":";
      put_u64(o, r.output_tokens);
      o += ",\"duration_ms\":";
      put_u64(o, r.duration_ms);
      o += ",\"prefill_tok_s\":";
      put_f64(o, r.prefill_tok_s);
      o += ",\"decode_tok_s\":";
      put_f64(o, r.decode_tok_s);
      o += ",\"status\":";
      put_str(o, r.status);
      o += "}";
    }
    o += "],\"settings\":{";
    bool first = true;
    for (const auto& kv : settings) {
      if (!first) o += ",";
      first = false;
      put_str(o, kv.first);
      o += ":";
      put_str(o, kv.second);
    }
    o += "},\"events\":[";
    for (size_t i = 0; i < events.size(); i++) {
      const Event& e = events[i];
      o += i ? ",{\"ts_ms\":" : "{\"ts_ms\":";
      put_u64(o, e.ts_ms);
      o += ",\"level\":";
      put_str(o, e.level);
      o += ",\"message\":";
      put_str(o, e.message);
      o += "}";
    }
    o += "]}";
    return o;
  }

  // Publisher::publish (snapshot.rs:172-185): the temporary file is written and its data synced before the rename,
  // so that a reader never sees half a file; a failed write leaves the previous file in place
  int publish() {
    const std::string s = json(now_ms());
    const int fd = open(tmp.c_str(), O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0600);
    if (fd < 0) return set_error(MOERT_E_CONFIG, "metrics: cannot create %s: %s", tmp.c_str(), strerror(errno));
    size_t off = 0;
    while (off < s.size()) {
      const ssize_t w = write(fd, s.data() + off, s.size() - off);
      if (w < 0 && errno == EINTR) continue;
      if (w <= 0) {
        const int e = errno;
        close(fd);
        unlink(tmp.c_str());
        return set_error(MOERT_E_CONFIG, "metrics: write to %s failed: %s", tmp.c_str(), strerror(e));
      }
      off += (size_t)w;
    }
    if (fdatasync(fd) != 0 || close(fd) != 0) {
      const int e = errno;
      unlink(tmp.c_str());
      return set_error(MOERT_E_CONFIG, "metrics: sync of %s failed: %s", tmp.c_str(), strerror(e));
    }
    if (rename(tmp.c_str(), path.c_str()) != 0) {
      const int e = errno;
      unlink(tmp.c_str());
      return set_error(MOERT_E_CONFIG, "metrics: rename to %s failed: %s", path.c_str(), strerror(e));
    }
    return MOERT_OK;
  }
};

#define MX_OK(mx) \
  if (!(mx)) return set_error(MOERT_E_CONFIG, "null metrics handle")

extern "C" {

int moert_metrics_create(const char* path, moert_metrics** out) {
  if (!out) return set_error(MOERT_E_CONFIG, "metrics: null output");
  *out = nullptr;
  std::string p = path && *path ? std::string(path) : default_path();
  if (p.back() == '/') return set_error(MOERT_E_CONFIG, "metrics: %s names a directory", p.c_str());
  std::string err;
  if (!make_parent_dirs(p, &err)) return set_error(MOERT_E_CONFIG, "metrics: cannot create directory %s", err.c_str());
  moert_metrics* mx = new moert_metrics();
  mx->path = p;
  // Path::with_extension("json.tmp-<pid>") on metrics.json
  const size_t slash = p.rfind('/'), dot = p.rfind('.');
  const std::string stem = dot != std::string::npos && (slash == std::string::npos || dot > slash + 1) ? p.substr(0, dot) : p;
  mx->pid = (uint32_t)getpid();
  mx->tmp = stem + ".json.tmp-" + std::to_string(mx->pid);
  mx->started_ms = now_ms();
  *out = mx;
  return MOERT_OK;
}

int moert_metrics_destroy(moert_metrics* mx) {
  delete mx;
  return MOERT_OK;
}

int moert_metrics_path(const moert_metrics* mx, char* buf, int len) {
  MX_OK(mx);
  if (!buf || len < 1) return set_error(MOERT_E_CONFIG, "metrics: empty path buffer");
  snprintf(buf, (size_t)len, "%s", mx->path.c_str());
  return MOERT_OK;
}

int moert_metrics_set_model(moert_metrics* mx, const char* name, int layers, int experts, int experts_per_tok) {
  MX_OK(mx);
  if (layers < 0 || experts < 0 || experts_per_tok < 0) return set_error(MOERT_E_CONFIG, "metrics: negative model size");
  std::lock_guard<std::mutex> l(mx->mu);
  mx->name = name ? name : "";
  mx->layers = (uint32_t)layers;
  mx->experts = (uint32_t)experts;
  mx->experts_per_tok = (uint32_t)experts_per_tok;
  return MOERT_OK;
}

int moert_metrics_set_state(moert_metrics* mx, int kind, uint64_t a, uint64_t b, const char* message) {
  MX_OK(mx);
  if (kind < MOERT_STATE_IDLE || kind > MOERT_STATE_ERROR) return set_error(MOERT_E_CONFIG, "metrics: state %d", kind);
  std::lock_guard<std::mutex> l(mx->mu);
  mx->state = kind;
  mx->sa = a;
  mx->sb = b;
  mx->message = message ? message : "";
  return MOERT_OK;
}

int moert_metrics_set_speed(moert_metrics* mx, const moert_metrics_speed* s) {
  MX_OK(mx);
  if (!s) return set_error(MOERT_E_CONFIG, "metrics: null speed");
  std::lock_guard<std::mutex> l(mx->mu);
  mx->speed = *s;
  return MOERT_OK;
}

int moert_metrics_set_context(moert_metrics* mx, uint64_t used, uint64_t max) {
  MX_OK(mx);
  std::lock_guard<std::mutex> l(mx->mu);
  mx->ctx_used = used;
  mx->ctx_max = max;
  return MOERT_OK;
}

int moert_metrics_set_cache(moert_metrics* mx, const moert_metrics_cache* c) {
  MX_OK(mx);
  if (!c) return set_error(MOERT_E_CONFIG, "metrics: null cache section");
  std::lock_guard<std::mutex> l(mx->mu);
  mx->cache = *c;
  return MOERT_OK;
}

int moert_metrics_set_window(moert_metrics* mx, const moert_metrics_window* w) {
  MX_OK(mx);
  if (!w) return set_error(MOERT_E_CONFIG, "metrics: null window");
  std::lock_guard<std::mutex> l(mx->mu);
  mx->window = *w;
  return MOERT_OK;
}

int moert_metrics_add_request(moert_metrics* mx, const moert_metrics_request* r) {
  MX_OK(mx);
  if (!r) return set_error(MOERT_E_CONFIG, "metrics: null request");
  std::lock_guard<std::mutex> l(mx->mu);
  mx->requests.push_front({r->started_ms, r->prompt_tokens, r->reused_tokens, r->output_tokens, r->duration_ms,
                           r->prefill_tok_s, r->decode_tok_s, r->status ? r->status : ""});
  while (mx->requests.size() > kMaxRequests) mx->requests.pop_back();
  return MOERT_OK;
}

int moert_metrics_setting(moert_metrics* mx, const char* key, const char* value) {
  MX_OK(mx);
  if (!key) return set_error(MOERT_E_CONFIG, "metrics: null setting name");
  std::lock_guard<std::mutex> l(mx->mu);
  mx->settings[key] = value ? value : "";
  return MOERT_OK;
}

int moert_metrics_event(moert_metrics* mx, const char* level, const char* message) {
  MX_OK(mx);
  std::lock_guard<std::mutex> l(mx->mu);
  mx->events.push_back({now_ms(), level ? level : "info", message ? message : ""});
  while (mx->events.size() > kMaxEvents) mx->events.pop_front();
  return MOERT_OK;
}

int moert_metrics_json(moert_metrics* mx, char* buf, size_t len, size_t* needed) {
  MX_OK(mx);
  std::string s;
  {
    std::lock_guard<std::mutex> l(mx->mu);
    s = mx->json(now_ms());
  }
  if (needed) *needed = s.size() + 1;
  if (buf && len > s.size()) memcpy(buf, s.c_str(), s.size() + 1);
  return MOERT_OK;
}

int moert_metrics_publish(moert_metrics* mx) {
  MX_OK(mx);
  std::lock_guard<std::mutex> l(mx->mu);
  return mx->publish();
}

}  // extern "C"
