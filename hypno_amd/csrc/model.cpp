// `.hypno` model files: read-only mapping, manifest parsing and a one-time,
// pipelined upload of every tensor payload to HBM (declared in
// include/hypno_hip.h).
//
// Parsing follows HypnoModel::open (loader.rs:39-134) field by field: the
// 16-byte header (format.rs:13-24, validated as format.rs:36-44), the
// metadata key/value pairs (loader.rs:57-90) and the tensor table
// (loader.rs:92-122), with the same checks in the same order and one
// FormatError variant (format.rs:109-131) per failure.  Where the reference
// reads without a bounds check (a tensor name's bytes, loader.rs:96-97) this
// reader reports BufferTooShort instead of reading past the mapping.
//
// Upload: the payload span [lowest offset rounded down to 64, highest end) is
// copied into one device allocation, so every tensor keeps its in-file
// alignment (64 bytes for files written by sft_convert.rs:140-168).  Four
// reader threads pread() 4 MiB pieces of the file into their own pair of
// pinned buffers and queue each piece's host-to-device copy on their own
// stream, so file reads, PCIe copies and the next reads overlap.  The pinned
// buffers, streams and events form a per-device staging pool created on the
// first upload and kept for the life of the process (32 MiB of pinned host
// memory per device): pinning and first-touching fresh buffers on every open
// cost more than the copy itself.  Uploads to one device are serialised on
// that pool.
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/hypno_hip.h"
#include "common.hpp"

struct hypno_hip_model {
  int fd = -1;
  const uint8_t* map = nullptr;  // read-only mapping of the whole file
  size_t size = 0;
  uint8_t magic[4] = {0, 0, 0, 0};
  uint32_t version = 0, kv_count = 0, tensor_count = 0;
  std::vector<std::string> keys, values;
  struct Tensor {
    std::string name;
    std::vector<uint64_t> shape;
    uint32_t ndim = 0, dtype = 0;
    uint64_t offset = 0, data_len = 0;
  };
  std::vector<Tensor> tensors;
  int device = -1;
  uint8_t* dev = nullptr;  // payload span on `device`, or NULL
  uint64_t dev_lo = 0, dev_len = 0;
};

namespace {

using hypno::set_last_error;

constexpr uint8_t kMagic[4] = {0x48, 0x59, 0x50, 0x4E};  // "HYPN" (format.rs:4)
constexpr uint32_t kFormatVersion = 1;                    // format.rs:7
constexpr uint64_t kAlignment = 64;                       // format.rs:10
constexpr size_t kPiece = 4u << 20;                       // upload piece
constexpr int kReaders = 4;

int format_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
int format_error(const char* fmt, ...) {
  char buf[256];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  return set_last_error(HYPNO_HIP_EFORMAT, buf);
}

int too_short(size_t needed, size_t got) {
  return format_error("buffer too short: needed %zu bytes, got %zu", needed, got);
}

// std::str::from_utf8: well-formed UTF-8 only (no overlong forms, no
// surrogates, nothing above U+10FFFF).  Returns the index of the first bad
// byte, or len.
size_t utf8_valid_up_to(const uint8_t* s, size_t len) {
  size_t i = 0;
  while (i < len) {
    const uint8_t c = s[i];
    if (c < 0x80) {
      i++;
      continue;
    }
    size_t n;
    uint8_t lo = 0x80, hi = 0xBF;
    if (c >= 0xC2 && c <= 0xDF) {
      n = 1;
    } else if (c >= 0xE0 && c <= 0xEF) {
      n = 2;
      if (c == 0xE0) lo = 0xA0;
      if (c == 0xED) hi = 0x9F;
    } else if (c >= 0xF0 && c <= 0xF4) {
      n = 3;
      if (c == 0xF0) lo = 0x90;
      if (c == 0xF4) hi = 0x8F;
    } else {
      return i;
    }
    if (i + n >= len) return i;  // truncated sequence
    if (s[i + 1] < lo || s[i + 1] > hi) return i;
    for (size_t k = 2; k <= n; k++)
      if (s[i + k] < 0x80 || s[i + k] > 0xBF) return i;
    i += n + 1;
  }
  return len;
}

uint32_t rd32(const uint8_t* p) {
  uint32_t v;
  std::memcpy(&v, p, 4);  // little-endian host (x86-64)
  return v;
}

uint64_t rd64(const uint8_t* p) {
  uint64_t v;
  std::memcpy(&v, p, 8);
  return v;
}

// A length-prefixed UTF-8 string at `cur` whose length was just read.
int read_str(const uint8_t* d, size_t size, size_t& cur, size_t len, std::string& out) {
  if (len > size - cur) return too_short(cur + len, size);
  const size_t ok = utf8_valid_up_to(d + cur, len);
  if (ok != len)
    return format_error("UTF-8 error: invalid utf-8 at byte %zu of a %zu-byte string", ok, len);
  out.assign(reinterpret_cast<const char*>(d + cur), len);
  cur += len;
  return HYPNO_HIP_OK;
}

int read_u32(const uint8_t* d, size_t size, size_t& cur, uint32_t& v) {
  if (size - cur < 4) return too_short(cur + 4, size);
  v = rd32(d + cur);
  cur += 4;
  return HYPNO_HIP_OK;
}

int read_u64(const uint8_t* d, size_t size, size_t& cur, uint64_t& v) {
  if (size - cur < 8) return too_short(cur + 8, size);
  v = rd64(d + cur);
  cur += 8;
  return HYPNO_HIP_OK;
}

// HypnoModel::open after the mapping (loader.rs:44-134).
int parse(hypno_hip_model* m) {
  const uint8_t* d = m->map;
  const size_t size = m->size;
  if (size < 16) return too_short(16, size);
  std::memcpy(m->magic, d, 4);
  m->version = rd32(d + 4);
  m->kv_count = rd32(d + 8);
  m->tensor_count = rd32(d + 12);
  if (std::memcmp(m->magic, kMagic, 4) != 0)
    return format_error("invalid magic bytes: expected '[72, 89, 80, 78]', got '[%u, %u, %u, %u]'",
                        m->magic[0], m->magic[1], m->magic[2], m->magic[3]);
  if (m->version != kFormatVersion)
    return format_error("unsupported format version %u (expected 1)", m->version);
  size_t cur = 16;
  int st;
  // Every entry takes at least 4 bytes, so counts beyond size/4 fail below;
  // reserve no more than that.
  const size_t cap = size / 4;
  m->keys.reserve(std::min<size_t>(m->kv_count, cap));
  m->values.reserve(std::min<size_t>(m->kv_count, cap));
  for (uint32_t i = 0; i < m->kv_count; i++) {
    uint32_t kl, vl;
    std::string k, v;
    if ((st = read_u32(d, size, cur, kl)) || (st = read_str(d, size, cur, kl, k)) ||
        (st = read_u32(d, size, cur, vl)) || (st = read_str(d, size, cur, vl, v)))
      return st;
    m->keys.push_back(std::move(k));
    m->values.push_back(std::move(v));
  }
  m->tensors.reserve(std::min<size_t>(m->tensor_count, cap));
  for (uint32_t i = 0; i < m->tensor_count; i++) {
    hypno_hip_model::Tensor t;
    uint32_t nl;
    if ((st = read_u32(d, size, cur, nl)) || (st = read_str(d, size, cur, nl, t.name)) ||
        (st = read_u32(d, size, cur, t.ndim)))
      return st;
    for (uint32_t k = 0; k < t.ndim; k++) {
      uint64_t dim;
      if ((st = read_u64(d, size, cur, dim))) return st;
      t.shape.push_back(dim);
    }
    if ((st = read_u32(d, size, cur, t.dtype))) return st;
    if (t.dtype > HYPNO_DTYPE_Q4_0) return format_error("unknown dtype code: %u", t.dtype);
    if ((st = read_u64(d, size, cur, t.offset)) || (st = read_u64(d, size, cur, t.data_len)))
      return st;
    // offset + data_len > file_size, without wrapping (loader.rs:113-115).
    if (t.offset > size || t.data_len > size - t.offset)
      return format_error("invalid tensor offset %llu: out of file bounds (%zu)",
                          (unsigned long long)t.offset, size);
    m->tensors.push_back(std::move(t));
  }
  return HYPNO_HIP_OK;
}

int map_file(hypno_hip_model* m, const char* path) {
  m->fd = ::open(path, O_RDONLY | O_CLOEXEC);
  if (m->fd < 0) {
    const int err = errno;
    return set_last_error(err == ENOENT ? HYPNO_HIP_ENOENT : HYPNO_HIP_EFILE,
                          std::string("I/O error: open ") + path + ": " + std::strerror(err));
  }
  struct stat sb;
  if (fstat(m->fd, &sb) != 0)
    return set_last_error(HYPNO_HIP_EFILE, std::string("I/O error: fstat: ") + std::strerror(errno));
  if (!S_ISREG(sb.st_mode))
    return set_last_error(HYPNO_HIP_EFILE, std::string("I/O error: not a regular file: ") + path);
  m->size = (size_t)sb.st_size;
  if (m->size == 0) return HYPNO_HIP_OK;  // an empty mapping; parse() reports it
  void* p = mmap(nullptr, m->size, PROT_READ, MAP_PRIVATE, m->fd, 0);
  if (p == MAP_FAILED)
    return set_last_error(HYPNO_HIP_EFILE, std::string("I/O error: mmap: ") + std::strerror(errno));
  m->map = static_cast<const uint8_t*>(p);
  return HYPNO_HIP_OK;
}

void release(hypno_hip_model* m) {
  if (m->dev) (void)hipFree(m->dev);
  if (m->map) munmap(const_cast<uint8_t*>(m->map), m->size);
  if (m->fd >= 0) ::close(m->fd);
  delete m;
}

// One reader's pinned buffers, events and stream (on the pool's device).
struct Reader {
  void* buf[2] = {nullptr, nullptr};
  hipEvent_t done[2] = {nullptr, nullptr};
  hipStream_t stream = nullptr;
};

struct Staging {
  std::mutex mu;  // held for a whole upload
  bool ready = false;
  Reader r[kReaders];
};

std::mutex g_staging_mu;
std::map<int, std::unique_ptr<Staging>> g_staging;

void staging_free(Staging* sg) {
  for (Reader& r : sg->r) {
    for (int k = 0; k < 2; k++) {
      if (r.done[k]) (void)hipEventDestroy(r.done[k]);
      if (r.buf[k]) (void)hipHostFree(r.buf[k]);
      r.done[k] = nullptr;
      r.buf[k] = nullptr;
    }
    if (r.stream) (void)hipStreamDestroy(r.stream);
    r.stream = nullptr;
  }
}

// Create the pool on the current device (default-priority streams).
int staging_setup(Staging* sg) {
  for (Reader& r : sg->r) {
    hipError_t e = hipStreamCreateWithFlags(&r.stream, hipStreamNonBlocking);
    for (int k = 0; k < 2 && e == hipSuccess; k++) {
      e = hipHostMalloc(&r.buf[k], kPiece, hipHostMallocDefault);
      if (e == hipSuccess) {
        std::memset(r.buf[k], 0, kPiece);  // fault the pages in now, not mid-upload
        e = hipEventCreateWithFlags(&r.done[k], hipEventDisableTiming);
      }
    }
    if (e != hipSuccess) {
      staging_free(sg);
      return hypno::hip_status(e, "model upload: staging pool");
    }
  }
  sg->ready = true;
  return HYPNO_HIP_OK;
}

int upload(hypno_hip_model* m) {
  uint64_t lo = UINT64_MAX, hi = 0;
  for (const auto& t : m->tensors) {
    if (t.data_len == 0) continue;
    lo = std::min(lo, t.offset);
    hi = std::max(hi, t.offset + t.data_len);
  }
  if (hi == 0) return HYPNO_HIP_OK;  // no payload bytes
  lo -= lo % kAlignment;
  hipError_t e = hipGetDevice(&m->device);
  if (e != hipSuccess) return hypno::hip_status(e, "model upload: hipGetDevice");
  Staging* sg;
  {
    std::lock_guard<std::mutex> g(g_staging_mu);
    std::unique_ptr<Staging>& slot = g_staging[m->device];
    if (!slot) slot.reset(new Staging);
    sg = slot.get();
  }
  std::lock_guard<std::mutex> pool_lock(sg->mu);
  if (!sg->ready) {
    const int st = staging_setup(sg);
    if (st) return st;
  }
  m->dev_lo = lo;
  m->dev_len = hi - lo;
  e = hipMalloc(&m->dev, m->dev_len);
  if (e != hipSuccess) {
    m->dev = nullptr;
    return hypno::hip_status(e, "model upload: hipMalloc of the payload span");
  }
  const size_t pieces = (size_t)((m->dev_len + kPiece - 1) / kPiece);
  const int nthreads = (int)std::min<size_t>(pieces, kReaders);
  std::atomic<size_t> next{0};
  std::atomic<int> status{HYPNO_HIP_OK};
  std::vector<std::string> errors(nthreads);
  auto work = [&](int id) {
    Reader& r = sg->r[id];
    auto bail = [&](int st, const std::string& msg) {
      int expect = HYPNO_HIP_OK;
      if (status.compare_exchange_strong(expect, st)) errors[id] = msg;
    };
    auto hip_ok = [&](hipError_t err, const char* what) {
      if (err == hipSuccess) return true;
      bail(err == hipErrorOutOfMemory ? HYPNO_HIP_ENOMEM : HYPNO_HIP_EDEVICE,
           std::string("model upload: ") + what + ": " + hipGetErrorString(err));
      return false;
    };
    bool used[2] = {false, false};
    bool ok = hip_ok(hipSetDevice(m->device), "hipSetDevice");
    for (int k = 0; ok && status.load() == HYPNO_HIP_OK; k ^= 1) {
      const size_t i = next.fetch_add(1);
      if (i >= pieces) break;
      const uint64_t off = (uint64_t)i * kPiece;
      const size_t len = (size_t)std::min<uint64_t>(kPiece, m->dev_len - off);
      // The buffer's previous copy must be done before it is refilled.
      if (used[k] && !hip_ok(hipEventSynchronize(r.done[k]), "copy")) break;
      uint8_t* dst = static_cast<uint8_t*>(r.buf[k]);
      size_t got = 0;
      while (got < len) {
        const ssize_t n = pread(m->fd, dst + got, len - got, (off_t)(m->dev_lo + off + got));
        if (n < 0 && errno == EINTR) continue;
        if (n <= 0) {
          bail(HYPNO_HIP_EFILE, std::string("I/O error: pread: ") +
                                    (n < 0 ? std::strerror(errno) : "unexpected end of file"));
          ok = false;
          break;
        }
        got += (size_t)n;
      }
      if (!ok) break;
      ok = hip_ok(hipMemcpyAsync(m->dev + off, dst, len, hipMemcpyHostToDevice, r.stream),
                  "hipMemcpyAsync") &&
           hip_ok(hipEventRecord(r.done[k], r.stream), "event record");
      used[k] = true;
    }
    // Drain this reader's copies whatever happened: the pool's buffers are
    // reused by the next upload.
    hip_ok(hipStreamSynchronize(r.stream), "copy");
  };
  std::vector<std::thread> threads;
  for (int i = 1; i < nthreads; i++) threads.emplace_back(work, i);
  work(0);
  for (auto& t : threads) t.join();
  const int st = status.load();
  if (st != HYPNO_HIP_OK) {
    for (const auto& msg : errors)
      if (!msg.empty()) return set_last_error(st, msg);
    return set_last_error(st, "model upload failed");
  }
  return HYPNO_HIP_OK;
}

void fill_info(const hypno_hip_model* m, size_t i, hypno_hip_tensor_info* out) {
  const auto& t = m->tensors[i];
  out->name = t.name.c_str();
  out->dtype = t.dtype;
  out->ndim = t.ndim;
  out->shape = t.shape.empty() ? nullptr : t.shape.data();
  out->offset = t.offset;
  out->data_len = t.data_len;
  out->host = m->map ? m->map + t.offset : nullptr;
  out->device = (m->dev && t.data_len) ? m->dev + (t.offset - m->dev_lo) : nullptr;
}

}  // namespace

extern "C" {

int hypno_hip_model_open(const char* path, uint32_t flags, hypno_hip_model** model) {
  if (!path || !model) return set_last_error(HYPNO_HIP_EINVAL, "model_open: NULL argument");
  *model = nullptr;
  if (flags & ~HYPNO_HIP_MODEL_HOST_ONLY)
    return set_last_error(HYPNO_HIP_EINVAL, "model_open: unknown flag bits");
  hypno_hip_model* m = new (std::nothrow) hypno_hip_model;
  if (!m) return set_last_error(HYPNO_HIP_ENOMEM, "model_open: out of host memory");
  int st = map_file(m, path);
  if (!st) st = parse(m);
  if (!st && !(flags & HYPNO_HIP_MODEL_HOST_ONLY)) st = upload(m);
  if (st) {
    release(m);
    return st;
  }
  *model = m;
  return HYPNO_HIP_OK;
}

int hypno_hip_model_close(hypno_hip_model* model) {
  if (!model) return set_last_error(HYPNO_HIP_EINVAL, "model_close: NULL model");
  release(model);
  return HYPNO_HIP_OK;
}

int hypno_hip_model_header(const hypno_hip_model* m, uint32_t* version, uint32_t* metadata_kv_count,
                           uint32_t* tensor_count) {
  if (!m) return set_last_error(HYPNO_HIP_EINVAL, "model_header: NULL model");
  if (version) *version = m->version;
  if (metadata_kv_count) *metadata_kv_count = m->kv_count;
  if (tensor_count) *tensor_count = m->tensor_count;
  return HYPNO_HIP_OK;
}

int hypno_hip_model_metadata_at(const hypno_hip_model* m, size_t i, const char** key,
                                const char** value) {
  if (!m || !key || !value) return set_last_error(HYPNO_HIP_EINVAL, "metadata_at: NULL argument");
  if (i >= m->keys.size()) return set_last_error(HYPNO_HIP_EINVAL, "metadata_at: index out of range");
  *key = m->keys[i].c_str();
  *value = m->values[i].c_str();
  return HYPNO_HIP_OK;
}

int hypno_hip_model_metadata(const hypno_hip_model* m, const char* key, const char** value) {
  if (!m || !key || !value) return set_last_error(HYPNO_HIP_EINVAL, "metadata: NULL argument");
  *value = nullptr;
  for (size_t i = 0; i < m->keys.size(); i++)
    if (m->keys[i] == key) {  // first match (loader.rs:158-163)
      *value = m->values[i].c_str();
      return HYPNO_HIP_OK;
    }
  return set_last_error(HYPNO_HIP_ENOENT, std::string("metadata: no key ") + key);
}

int hypno_hip_model_tensor_at(const hypno_hip_model* m, size_t i, hypno_hip_tensor_info* out) {
  if (!m || !out) return set_last_error(HYPNO_HIP_EINVAL, "tensor_at: NULL argument");
  if (i >= m->tensors.size()) return set_last_error(HYPNO_HIP_EINVAL, "tensor_at: index out of range");
  fill_info(m, i, out);
  return HYPNO_HIP_OK;
}

int hypno_hip_model_find_tensor(const hypno_hip_model* m, const char* name,
                                hypno_hip_tensor_info* out) {
  if (!m || !name || !out) return set_last_error(HYPNO_HIP_EINVAL, "find_tensor: NULL argument");
  for (size_t i = 0; i < m->tensors.size(); i++)
    if (m->tensors[i].name == name) {  // first match (loader.rs:139-156)
      fill_info(m, i, out);
      return HYPNO_HIP_OK;
    }
  return set_last_error(HYPNO_HIP_ENOENT, std::string("find_tensor: no tensor ") + name);
}

int hypno_hip_model_is_col_major(const hypno_hip_model* m) {
  if (!m) return 0;
  for (size_t i = 0; i < m->keys.size(); i++)
    if (m->keys[i] == "weight_layout") return m->values[i] == "col_major";  // loader.rs:166-168
  return 0;
}

}  // extern "C"
