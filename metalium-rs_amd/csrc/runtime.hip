// Context, buffer table, caching allocator, pinned host transfers, the
// sticky asynchronous error, events and the op report.
//
// Reference: the device server (crates/burn-tt/src/server.rs) -- attach and
// the engine (2738, 4071), `DramBuffers` (868), upload/download through a
// pinned staging page (crates/tt-kernels/src/session.rs:4128, 4225, 4295,
// 4741), the deferred failure reported at the next wait (2951-2991) -- and the
// op report (crates/burn-tt/src/report.rs:29-51).
#include "common.hpp"

#include <atomic>
#include <new>

namespace mi {

static thread_local std::string g_global_error;
static std::atomic<uint64_t> g_next_id{1};  // ids are never reused

const char *elem_name(int elem) {
  switch (elem) {
    case MI_F32: return "F32";
    case MI_I32: return "I32";
    case MI_BOOL: return "Bool";
    case MI_BF16: return "BF16";
    case MI_BFP8: return "BFP8";
    default: return "?";
  }
}

int fail(Ctx *ctx, int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (ctx) ctx->last_error = buf; else g_global_error = buf;
  return code;
}

int check_launch(Ctx *ctx, const char *what) {
  hipError_t e = hipGetLastError();
  ctx->report.ops++;
  if (e != hipSuccess) {
    int code = fail(ctx, MI_E_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
    if (ctx->sticky == MI_OK) { ctx->sticky = code; ctx->sticky_msg = ctx->last_error; }
    return code;
  }
  return MI_OK;
}

Buffer *lookup(Ctx *ctx, mi_id id) {
  auto it = ctx->bufs.find(id);
  return it == ctx->bufs.end() ? nullptr : &it->second;
}

mi_id insert(Ctx *ctx, const Buffer &b) {
  mi_id id = g_next_id.fetch_add(1);
  ctx->bufs.emplace(id, b);
  ctx->live_bytes += b.bytes;
  return id;
}

static size_t round_size(size_t bytes) {
  if (bytes == 0) bytes = 1;
  if (bytes <= (size_t(1) << 20)) return (bytes + 511) & ~size_t(511);
  return (bytes + (size_t(2) << 20) - 1) & ~((size_t(2) << 20) - 1);
}

void *device_alloc(Ctx *ctx, size_t bytes, size_t *got) {
  size_t sz = round_size(bytes);
  if (ctx->capturing) {
    // A block this capture freed: it leaves the trace's held list while the
    // capture's new buffer has it (mi_free returns it there).
    auto cf = ctx->capture_free.find(sz);
    if (cf != ctx->capture_free.end() && !cf->second.empty()) {
      void *p = cf->second.back();
      cf->second.pop_back();
      auto &held = ctx->traces[ctx->capture_id].held;
      for (size_t i = 0; i < held.size(); ++i)
        if (held[i].first == p) {
          held[i] = held.back();
          held.pop_back();
          break;
        }
      *got = sz;
      return p;
    }
  }
  auto it = ctx->free_blocks.find(sz);
  if (it != ctx->free_blocks.end() && !it->second.empty()) {
    void *p = it->second.back();
    it->second.pop_back();
    ctx->cached_bytes -= sz;
    *got = sz;
    return p;
  }
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, sz);
  if (e != hipSuccess && ctx->capturing) {
    (void)hipGetLastError();  // no wait is possible inside a capture
    return nullptr;
  }
  if (e != hipSuccess) {
    // Give the cache back to the device and try once more.
    (void)hipGetLastError();
    (void)hipStreamSynchronize(ctx->stream);
    for (auto &kv : ctx->free_blocks)
      for (void *q : kv.second) (void)hipFree(q);
    ctx->free_blocks.clear();
    ctx->cached_bytes = 0;
    e = hipMalloc(&p, sz);
    if (e != hipSuccess) { (void)hipGetLastError(); return nullptr; }
  }
  *got = sz;
  return p;
}

void device_release(Ctx *ctx, void *p, size_t bytes) {
  if (!p) return;
  ctx->free_blocks[bytes].push_back(p);
  ctx->cached_bytes += bytes;
}

int new_buffer(Ctx *ctx, int64_t rows, int64_t cols, int elem, mi_id *id, Buffer **out) {
  if (rows < 0 || cols < 0) return fail(ctx, MI_E_ARG, "negative dims [%lld, %lld]", (long long)rows, (long long)cols);
  if (!elem_valid(elem)) return fail(ctx, MI_E_ARG, "unknown element kind %d", elem);
  Buffer b;
  b.rows = rows; b.cols = cols; b.elem = elem;
  b.trace = ctx->capturing ? ctx->capture_id : 0;
  size_t want = storage_bytes(elem, rows, cols);
  b.ptr = device_alloc(ctx, want, &b.bytes);
  if (!b.ptr) return fail(ctx, MI_E_OOM, "device allocation of %zu bytes failed", want);
  *id = insert(ctx, b);
  if (out) *out = lookup(ctx, *id);
  return MI_OK;
}

void *scratch(Ctx *ctx, size_t bytes) {
  if (bytes <= ctx->scratch_bytes) return ctx->scratch;
  if (ctx->scratch) {
    if (ctx->capturing || !ctx->traces.empty()) {
      // A trace may replay kernels that use it: keep it until the context ends.
      ctx->retired_scratch.push_back(ctx->scratch);
    } else {
      // Earlier work on the stream may still read the old scratch.
      (void)hipStreamSynchronize(ctx->stream);
      (void)hipFree(ctx->scratch);
    }
  }
  size_t sz = round_size(bytes);
  if (hipMalloc(&ctx->scratch, sz) != hipSuccess) {
    (void)hipGetLastError();
    ctx->scratch = nullptr; ctx->scratch_bytes = 0;
    return nullptr;
  }
  ctx->scratch_bytes = sz;
  return ctx->scratch;
}

// Next staging slot, waiting for the copy that last used it.
static int stage_slot(Ctx *ctx) {
  int s = ctx->stage_next;
  ctx->stage_next = (s + 1) % Ctx::kStageSlots;
  if (ctx->stage_pending[s]) {
    (void)hipEventSynchronize(ctx->stage_done[s]);
    ctx->stage_pending[s] = false;
  }
  return s;
}

int refuse_if_capturing(Ctx *ctx, const char *what) {
  if (!ctx->capturing) return MI_OK;
  return fail(ctx, MI_E_UNSUPPORTED, "%s while a trace is being captured", what);
}

// Collect the device flags and stream errors into the sticky status.
static int collect(Ctx *ctx) {
  hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    int code = fail(ctx, MI_E_HIP, "stream failure: %s", hipGetErrorString(e));
    if (ctx->sticky == MI_OK) { ctx->sticky = code; ctx->sticky_msg = ctx->last_error; }
    return ctx->sticky;
  }
  uint32_t f = 0;
  e = hipMemcpy(&f, ctx->dev_flags, sizeof f, hipMemcpyDeviceToHost);
  if (e == hipSuccess && f != 0) {
    uint32_t zero = 0;
    (void)hipMemcpy(ctx->dev_flags, &zero, sizeof zero, hipMemcpyHostToDevice);
    if (ctx->sticky == MI_OK) {
      ctx->sticky = MI_E_DOMAIN;
      fail(ctx, MI_E_DOMAIN, (f & FLAG_INDEX_RANGE) ? "an index was out of range (DOMAIN)"
                                                    : "a value stored as BFP8 was not finite (DOMAIN)");
      ctx->sticky_msg = ctx->last_error;
    }
  }
  return ctx->sticky;
}

// Report and clear the sticky failure.
static int take_sticky(Ctx *ctx) {
  int s = ctx->sticky;
  if (s != MI_OK) {
    ctx->last_error = ctx->sticky_msg;
    ctx->sticky = MI_OK;
    ctx->sticky_msg.clear();
  }
  return s;
}

}  // namespace mi

using namespace mi;

extern "C" {

int mi_ctx_create(int device, mi_ctx **out) {
  if (!out) return fail(nullptr, MI_E_ARG, "null out pointer");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0) return fail(nullptr, MI_E_HIP, "no HIP device: %s", hipGetErrorString(e));
  if (device < 0 || device >= n) return fail(nullptr, MI_E_ARG, "device %d of %d", device, n);
  e = hipSetDevice(device);
  if (e != hipSuccess) return fail(nullptr, MI_E_HIP, "hipSetDevice(%d): %s", device, hipGetErrorString(e));
  mi_ctx *c = new (std::nothrow) mi_ctx();
  if (!c) return fail(nullptr, MI_E_OOM, "context allocation");
  c->device = device;
  // Messages up to fail()'s 512 bytes never allocate after this.
  c->last_error.reserve(512);
  c->sticky_msg.reserve(512);
  e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipMalloc(&c->dev_flags, 256);
  if (e == hipSuccess) e = hipMemset(c->dev_flags, 0, 256);
  for (int i = 0; e == hipSuccess && i < Ctx::kStageSlots; ++i) {
    e = hipHostMalloc(&c->stage[i], Ctx::kStageBytes, hipHostMallocDefault);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&c->stage_done[i], hipEventDisableTiming);
  }
  for (int i = 0; e == hipSuccess && i < 16; ++i) e = hipEventCreate(&c->events[i]);
  if (e != hipSuccess) {
    int code = fail(nullptr, MI_E_HIP, "context set-up: %s", hipGetErrorString(e));
    mi_ctx_destroy(c);
    return code;
  }
  // A failure here only disables mi_attention_rows_into, which reports it.
  (void)attention_scratch_setup(c);
  *out = c;
  return MI_OK;
}

int mi_ctx_destroy(mi_ctx *ctx) {
  if (!ctx) return MI_OK;
  {
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    for (auto &kv : ctx->bufs) (void)hipFree(kv.second.ptr);
    ctx->bufs.clear();
    for (auto &kv : ctx->free_blocks)
      for (void *p : kv.second) (void)hipFree(p);
    ctx->free_blocks.clear();
    if (ctx->capturing) {
      hipGraph_t g = nullptr;
      (void)hipStreamEndCapture(ctx->stream, &g);
      if (g) (void)hipGraphDestroy(g);
      (void)hipGetLastError();
    }
    for (auto &kv : ctx->traces) {
      if (kv.second.exec) (void)hipGraphExecDestroy(kv.second.exec);
      for (auto &h : kv.second.held) (void)hipFree(h.first);
    }
    ctx->traces.clear();
    for (void *p : ctx->retired_scratch) (void)hipFree(p);
    if (ctx->scratch) (void)hipFree(ctx->scratch);
    if (ctx->dev_flags) (void)hipFree(ctx->dev_flags);
    for (int i = 0; i < Ctx::kStageSlots; ++i) {
      if (ctx->stage[i]) (void)hipHostFree(ctx->stage[i]);
      if (ctx->stage_done[i]) (void)hipEventDestroy(ctx->stage_done[i]);
    }
    for (int i = 0; i < 16; ++i)
      if (ctx->events[i]) (void)hipEventDestroy(ctx->events[i]);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
  }
  delete ctx;
  return MI_OK;
}

const char *mi_last_error(const mi_ctx *ctx) {
  return ctx ? ctx->last_error.c_str() : g_global_error.c_str();
}

int mi_sync(mi_ctx *ctx) {
  MI_ENTER(ctx);
  if (int r = refuse_if_capturing(ctx, "sync")) return r;
  collect(ctx);
  return take_sticky(ctx);
}

int mi_stream(mi_ctx *ctx, void **stream) {
  MI_ENTER(ctx);
  if (!stream) return fail(ctx, MI_E_ARG, "null out pointer");
  *stream = ctx->stream;
  return MI_OK;
}

// Host bytes into an existing buffer through the pinned staging ring.
static int write_into(mi_ctx *ctx, Buffer *b, const void *src, size_t bytes) {
  const char *p = static_cast<const char *>(src);
  char *d = static_cast<char *>(b->ptr);
  for (size_t off = 0; off < bytes; off += Ctx::kStageBytes) {
    size_t n = std::min(Ctx::kStageBytes, bytes - off);
    int slot = stage_slot(ctx);
    std::memcpy(ctx->stage[slot], p + off, n);
    hipError_t e = hipMemcpyAsync(d + off, ctx->stage[slot], n, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipEventRecord(ctx->stage_done[slot], ctx->stream);
    if (e != hipSuccess) return fail(ctx, MI_E_HIP, "upload: %s", hipGetErrorString(e));
    ctx->stage_pending[slot] = true;
  }
  ctx->report.uploads++;
  ctx->report.bytes_up += bytes;
  return MI_OK;
}

static int upload_raw(mi_ctx *ctx, const void *src, int64_t rows, int64_t cols, int elem, mi_id *out) {
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  if (!src && rows * cols > 0) return fail(ctx, MI_E_ARG, "null host pointer");
  if (int r = refuse_if_capturing(ctx, "upload")) return r;
  if (elem == MI_BFP8) return fail(ctx, MI_E_ARG, "a BFP8 buffer is made on the device by mi_cast_bfp, not uploaded");
  mi_id id; Buffer *b;
  int s = new_buffer(ctx, rows, cols, elem, &id, &b);
  if (s) return s;
  s = write_into(ctx, b, src, static_cast<size_t>(rows * cols) * elem_size(elem));
  if (s) {
    mi_free(ctx, id);
    return s;
  }
  *out = id;
  return MI_OK;
}

int mi_upload(mi_ctx *ctx, const float *values, int64_t rows, int64_t cols, mi_id *out) {
  MI_ENTER(ctx);
  return upload_raw(ctx, values, rows, cols, MI_F32, out);
}

int mi_upload_bits(mi_ctx *ctx, const uint32_t *bits, int64_t rows, int64_t cols, int elem, mi_id *out) {
  MI_ENTER(ctx);
  if (elem == MI_BF16) return fail(ctx, MI_E_ARG, "BF16 takes mi_upload_bf16");
  return upload_raw(ctx, bits, rows, cols, elem, out);
}

int mi_upload_bf16(mi_ctx *ctx, const uint16_t *bits, int64_t rows, int64_t cols, mi_id *out) {
  MI_ENTER(ctx);
  return upload_raw(ctx, bits, rows, cols, MI_BF16, out);
}

static int download_raw(mi_ctx *ctx, mi_id id, void *dst, int64_t n, int want_elem_size, const char *what) {
  if (int r = refuse_if_capturing(ctx, what)) return r;
  MI_BUF(ctx, b, id);
  if (static_cast<int>(elem_size(b->elem)) != want_elem_size)
    return fail(ctx, MI_E_ARG, "%s of a %s buffer", what, elem_name(b->elem));
  if (n < b->numel()) return fail(ctx, MI_E_ARG, "%s: room for %lld of %lld datums", what, (long long)n, (long long)b->numel());
  // Wait for the producer; report an earlier failure first.
  int s = collect(ctx);
  if (s != MI_OK) return take_sticky(ctx);
  size_t bytes = static_cast<size_t>(b->numel()) * elem_size(b->elem);
  const char *d = static_cast<const char *>(b->ptr);
  char *o = static_cast<char *>(dst);
  // Up to kStageSlots chunks in flight: the copy of chunk k + slots is issued
  // as soon as chunk k has left its slot, so the device-to-host copies overlap
  // the host copies out of the staging memory.
  constexpr int S = Ctx::kStageSlots;
  const size_t nch = (bytes + Ctx::kStageBytes - 1) / Ctx::kStageBytes;
  int slot_of[S] = {};
  auto issue = [&](size_t k) -> hipError_t {
    const size_t off = k * Ctx::kStageBytes, m = std::min(Ctx::kStageBytes, bytes - off);
    const int slot = stage_slot(ctx);  // waits for the slot's previous copy
    slot_of[k % S] = slot;
    hipError_t e = hipMemcpyAsync(ctx->stage[slot], d + off, m, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipEventRecord(ctx->stage_done[slot], ctx->stream);
    if (e == hipSuccess) ctx->stage_pending[slot] = true;
    return e;
  };
  hipError_t e = hipSuccess;
  for (size_t k = 0; k < nch && k < static_cast<size_t>(S) && e == hipSuccess; ++k) e = issue(k);
  for (size_t k = 0; k < nch && e == hipSuccess; ++k) {
    const int slot = slot_of[k % S];
    e = hipEventSynchronize(ctx->stage_done[slot]);
    if (e != hipSuccess) break;
    ctx->stage_pending[slot] = false;
    const size_t off = k * Ctx::kStageBytes;
    std::memcpy(o + off, ctx->stage[slot], std::min(Ctx::kStageBytes, bytes - off));
    if (k + S < nch) e = issue(k + S);
  }
  if (e != hipSuccess) return fail(ctx, MI_E_HIP, "%s: %s", what, hipGetErrorString(e));
  ctx->report.downloads++;
  ctx->report.bytes_down += bytes;
  return MI_OK;
}

int mi_download(mi_ctx *ctx, mi_id id, float *out, int64_t n) {
  MI_ENTER(ctx);
  MI_BUF(ctx, b, id);
  if (b->elem == MI_BFP8) {  // its decoded values, as the reference's download_bfp
    if (int r = refuse_if_capturing(ctx, "download")) return r;
    if (n < b->numel())
      return fail(ctx, MI_E_ARG, "download: room for %lld of %lld datums", (long long)n, (long long)b->numel());
    mi_id t;
    if (int s = bfp8_decode_to(ctx, b, MI_F32, &t, nullptr)) return s;
    const int s = download_raw(ctx, t, out, n, 4, "download");
    mi_free(ctx, t);
    return s;
  }
  if (b->elem != MI_F32) return fail(ctx, MI_E_ARG, "download of a %s buffer as F32", elem_name(b->elem));
  return download_raw(ctx, id, out, n, 4, "download");
}

int mi_download_bits(mi_ctx *ctx, mi_id id, uint32_t *out, int64_t n) {
  MI_ENTER(ctx);
  return download_raw(ctx, id, out, n, 4, "download_bits");
}

int mi_download_bf16(mi_ctx *ctx, mi_id id, uint16_t *out, int64_t n) {
  MI_ENTER(ctx);
  return download_raw(ctx, id, out, n, 2, "download_bf16");
}

int mi_free(mi_ctx *ctx, mi_id id) {
  MI_ENTER(ctx);
  auto it = ctx->bufs.find(id);
  if (it == ctx->bufs.end()) return fail(ctx, MI_E_ID, "free of unknown buffer id %llu", (unsigned long long)id);
  ctx->live_bytes -= it->second.bytes;
  // While capturing, any freed memory may be referenced by the capture's
  // kernels: it is the capture's until the trace is released.
  const uint64_t owner = ctx->capturing ? ctx->capture_id : it->second.trace;
  auto tr = owner ? ctx->traces.find(owner) : ctx->traces.end();
  if (tr != ctx->traces.end()) {
    tr->second.held.emplace_back(it->second.ptr, it->second.bytes);  // the trace's until released
    if (ctx->capturing) ctx->capture_free[it->second.bytes].push_back(it->second.ptr);
  } else {
    device_release(ctx, it->second.ptr, it->second.bytes);
  }
  ctx->bufs.erase(it);
  return MI_OK;
}

int mi_metadata(mi_ctx *ctx, mi_id id, int64_t *rows, int64_t *cols, int *elem) {
  MI_ENTER(ctx);
  MI_BUF(ctx, b, id);
  if (rows) *rows = b->rows;
  if (cols) *cols = b->cols;
  if (elem) *elem = b->elem;
  return MI_OK;
}

int mi_reshape(mi_ctx *ctx, mi_id id, int64_t rows, int64_t cols) {
  MI_ENTER(ctx);
  MI_BUF(ctx, b, id);
  if (rows < 0 || cols < 0 || rows * cols != b->numel() || ((b->elem == MI_BFP8 || b->tiles) && cols != b->cols) ||
      (b->tiles && rows != b->rows))
    return fail(ctx, MI_E_ARG, "reshape of %s [%lld, %lld]%s to [%lld, %lld]", elem_name(b->elem), (long long)b->rows,
                (long long)b->cols, b->tiles ? " in tiles" : "", (long long)rows, (long long)cols);
  b->rows = rows;
  b->cols = cols;
  return MI_OK;
}

int mi_event_record(mi_ctx *ctx, int slot) {
  MI_ENTER(ctx);
  if (int r = refuse_if_capturing(ctx, "event record")) return r;
  if (slot < 0 || slot >= 16) return fail(ctx, MI_E_ARG, "event slot %d", slot);
  hipError_t e = hipEventRecord(ctx->events[slot], ctx->stream);
  return e == hipSuccess ? MI_OK : fail(ctx, MI_E_HIP, "event record: %s", hipGetErrorString(e));
}

int mi_event_elapsed_ms(mi_ctx *ctx, int from, int to, float *ms) {
  MI_ENTER(ctx);
  if (int r = refuse_if_capturing(ctx, "event wait")) return r;
  if (from < 0 || from >= 16 || to < 0 || to >= 16 || !ms) return fail(ctx, MI_E_ARG, "event slots %d %d", from, to);
  hipError_t e = hipEventSynchronize(ctx->events[to]);
  if (e == hipSuccess) e = hipEventElapsedTime(ms, ctx->events[from], ctx->events[to]);
  return e == hipSuccess ? MI_OK : fail(ctx, MI_E_HIP, "event elapsed: %s", hipGetErrorString(e));
}

int mi_copy_into(mi_ctx *ctx, mi_id src, mi_id dst) {
  MI_ENTER(ctx);
  MI_BUF(ctx, sb, src);
  MI_BUF(ctx, db, dst);
  const size_t n = sb->storage();
  if ((sb->elem == MI_BFP8) != (db->elem == MI_BFP8) ||
      (sb->elem == MI_BFP8 && (sb->rows != db->rows || sb->cols != db->cols)))
    return fail(ctx, MI_E_ARG, "copy_into: %s [%lld, %lld] into %s [%lld, %lld]", elem_name(sb->elem),
                (long long)sb->rows, (long long)sb->cols, elem_name(db->elem), (long long)db->rows, (long long)db->cols);
  if (n != db->storage()) return fail(ctx, MI_E_ARG, "copy_into: %zu bytes into %zu", n, db->storage());
  if (n > 0 && sb->ptr != db->ptr) {
    hipError_t e = hipMemcpyAsync(db->ptr, sb->ptr, n, hipMemcpyDeviceToDevice, ctx->stream);
    if (e != hipSuccess) return fail(ctx, MI_E_HIP, "copy_into: %s", hipGetErrorString(e));
  }
  return MI_OK;
}

int mi_trace_begin(mi_ctx *ctx) {
  MI_ENTER(ctx);
  if (ctx->capturing) return fail(ctx, MI_E_ARG, "a trace is already being captured");
  // Earlier asynchronous failures surface before the capture starts.
  collect(ctx);
  if (int s = take_sticky(ctx)) return s;
  hipError_t e = hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeRelaxed);
  if (e != hipSuccess) return fail(ctx, MI_E_HIP, "begin capture: %s", hipGetErrorString(e));
  ctx->capture_id = ctx->next_trace++;
  ctx->traces[ctx->capture_id] = Ctx::Trace{};
  ctx->capture_free.clear();
  ctx->capturing = true;
  return MI_OK;
}

int mi_trace_end(mi_ctx *ctx, uint64_t *trace) {
  MI_ENTER(ctx);
  if (!ctx->capturing) return fail(ctx, MI_E_ARG, "no trace is being captured");
  ctx->capturing = false;
  ctx->capture_free.clear();
  const uint64_t id = ctx->capture_id;
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(ctx->stream, &g);
  hipGraphExec_t exec = nullptr;
  if (e == hipSuccess) e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
  if (g) (void)hipGraphDestroy(g);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    mi_trace_release(ctx, id);
    return fail(ctx, MI_E_HIP, "end capture: %s", hipGetErrorString(e));
  }
  ctx->traces[id].exec = exec;
  if (trace) *trace = id;
  return MI_OK;
}

int mi_trace_run(mi_ctx *ctx, uint64_t trace, int64_t n_inputs, const mi_id *inputs, const void *const *values,
                 const int64_t *value_bytes, int64_t n_outputs, const mi_id *outputs, void *const *out_values,
                 const int64_t *out_bytes) {
  MI_ENTER(ctx);
  if (int r = refuse_if_capturing(ctx, "trace replay")) return r;
  auto it = ctx->traces.find(trace);
  if (it == ctx->traces.end() || !it->second.exec) return fail(ctx, MI_E_ID, "unknown trace %llu", (unsigned long long)trace);
  if (n_inputs < 0 || n_outputs < 0 || (n_inputs && (!inputs || !values || !value_bytes)) ||
      (n_outputs && (!outputs || !out_values || !out_bytes)))
    return fail(ctx, MI_E_ARG, "trace_run: input or output lists");
  // Every input's length and every output's room are checked before any
  // byte is written: an input's host bytes are its buffer's size exactly,
  // an output's room at least its buffer's size.
  for (int64_t i = 0; i < n_inputs; ++i) {
    MI_BUF(ctx, b, inputs[i]);
    const int64_t bytes = b->numel() * static_cast<int64_t>(elem_size(b->elem));
    if (!values[i]) return fail(ctx, MI_E_ARG, "trace_run: null values for input %lld", (long long)i);
    if (b->elem == MI_BFP8) return fail(ctx, MI_E_ARG, "trace_run: input %lld is a BFP8 buffer", (long long)i);
    if (value_bytes[i] != bytes)
      return fail(ctx, MI_E_ARG, "trace_run: input %lld is %lld bytes, its buffer %lld", (long long)i,
                  (long long)value_bytes[i], (long long)bytes);
  }
  for (int64_t i = 0; i < n_outputs; ++i) {
    MI_BUF(ctx, b, outputs[i]);
    const int64_t bytes = b->numel() * static_cast<int64_t>(elem_size(b->elem));
    if (!out_values[i]) return fail(ctx, MI_E_ARG, "trace_run: null destination for output %lld", (long long)i);
    if (b->elem == MI_BFP8) return fail(ctx, MI_E_ARG, "trace_run: output %lld is a BFP8 buffer", (long long)i);
    if (out_bytes[i] < bytes)
      return fail(ctx, MI_E_ARG, "trace_run: output %lld has room for %lld bytes of %lld", (long long)i,
                  (long long)out_bytes[i], (long long)bytes);
  }
  for (int64_t i = 0; i < n_inputs; ++i) {
    MI_BUF(ctx, b, inputs[i]);
    if (int s = write_into(ctx, b, values[i], static_cast<size_t>(value_bytes[i]))) return s;
  }
  hipError_t e = hipGraphLaunch(it->second.exec, ctx->stream);
  if (e != hipSuccess) return fail(ctx, MI_E_HIP, "trace launch: %s", hipGetErrorString(e));
  ctx->report.ops++;
  for (int64_t i = 0; i < n_outputs; ++i) {
    MI_BUF(ctx, b, outputs[i]);
    const int esz = static_cast<int>(elem_size(b->elem));
    if (int s = download_raw(ctx, outputs[i], out_values[i], out_bytes[i] / esz, esz, "trace output")) return s;
  }
  return MI_OK;
}

int mi_trace_release(mi_ctx *ctx, uint64_t trace) {
  MI_ENTER(ctx);
  auto it = ctx->traces.find(trace);
  if (it == ctx->traces.end()) return fail(ctx, MI_E_ID, "unknown trace %llu", (unsigned long long)trace);
  if (ctx->capturing && ctx->capture_id == trace) return fail(ctx, MI_E_ARG, "the trace is still being captured");
  // A replay may still be running: wait, then hand the memory back.
  (void)hipStreamSynchronize(ctx->stream);
  if (it->second.exec) (void)hipGraphExecDestroy(it->second.exec);
  for (auto &h : it->second.held) device_release(ctx, h.first, h.second);
  ctx->traces.erase(it);
  for (auto &kv : ctx->bufs)
    if (kv.second.trace == trace) kv.second.trace = 0;
  return MI_OK;
}

int mi_get_report(mi_ctx *ctx, mi_report *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  *out = ctx->report;
  out->live_buffers = ctx->bufs.size();
  out->device_bytes = ctx->live_bytes;
  out->cached_bytes = ctx->cached_bytes;
  return MI_OK;
}

}  // extern "C"
