// engref.cpp -- ENGREF01 reader and weight-slab uploader.
//
// Container layout (little-endian), as the reference writes and reads it
// (tools/gen_reference.py:56-83, tests/golden.hpp:21-33):
//   "ENGREF01" | int32 n_tensors | per tensor: int32 name_len, name bytes,
//   int32 dtype, int32 ndim, int64 dims[ndim], int64 n_bytes, data[n_bytes].
// The reference reader accepts dtype 0 (float32) only (tests/golden.cpp:105-109);
// this one also accepts 1 (IEEE binary16, stored at native size) and 2
// (float64). Validation order and messages follow tests/golden.cpp:108-194:
// magic, tensor count (0..4096), name length (1..1024), dtype, ndim (0..8),
// non-negative dims, n_bytes == numel * element size, complete data, unique
// names, no trailing bytes.
//
// The file is memory-mapped read-only and parsed in place: tensor data is
// never copied on the host until an upload. An upload places every tensor in
// one caller-owned device allocation (the slab) at 256-byte aligned offsets
// in file order, streaming the mapped bytes through two pinned staging
// buffers so the host copy of one chunk overlaps the DMA of the previous one.
#include "engine_internal.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstring>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

namespace {

constexpr char kMagic[8] = {'E', 'N', 'G', 'R', 'E', 'F', '0', '1'};
constexpr std::int32_t kMaxTensors = 4096;
constexpr std::int32_t kMaxNameLen = 1024;
constexpr std::int32_t kMaxNdim = 8;
constexpr std::int64_t kSlabAlign = 256;
constexpr std::size_t kStageBytes = 8u << 20;

struct TensorEntry {
  std::string name;
  std::int32_t dtype = 0;
  std::vector<std::int64_t> dims;
  std::int64_t nbytes = 0;
  std::size_t file_offset = 0;
  std::int64_t slab_offset = 0;
};

std::int64_t element_bytes(std::int32_t dtype) {
  switch (dtype) {
    case ENG_ENGREF_F32: return 4;
    case ENG_ENGREF_F16: return 2;
    case ENG_ENGREF_F64: return 8;
    default: return 0;
  }
}

}  // namespace

struct eng_engref_s {
  std::string path;
  const unsigned char* map = nullptr;
  std::size_t size = 0;
  std::vector<TensorEntry> tensors;
  std::unordered_map<std::string, std::int32_t> by_name;
  std::int64_t slab_bytes = 0;

  ~eng_engref_s() {
    if (map != nullptr) munmap(const_cast<unsigned char*>(map), size);
  }
};

namespace {

[[noreturn]] void bad_file(const std::string& path, const std::string& why) {
  eng::raise(ENG_INVALID_ARGUMENT, __FILE__, __LINE__, "engref file is well-formed",
             "engref file '" + path + "': " + why);
}

// Bounds-checked little-endian reads over the mapping.
class Cursor {
 public:
  Cursor(const eng_engref_s& f) : f_(f) {}

  template <typename T>
  T pod(const char* what) {
    T v{};
    if (f_.size - pos_ < sizeof(T)) {
      bad_file(f_.path, std::string("unexpected end of file while reading ") + what);
    }
    std::memcpy(&v, f_.map + pos_, sizeof(T));
    pos_ += sizeof(T);
    return v;
  }

  bool take(std::size_t n, std::size_t* start) {
    if (f_.size - pos_ < n) return false;
    *start = pos_;
    pos_ += n;
    return true;
  }

  std::size_t pos() const { return pos_; }

 private:
  const eng_engref_s& f_;
  std::size_t pos_ = 0;
};

void parse(eng_engref_s& f) {
  if (f.size < sizeof(kMagic) || std::memcmp(f.map, kMagic, sizeof(kMagic)) != 0) {
    bad_file(f.path, "bad magic -- not an ENGREF01 file");
  }
  Cursor c(f);
  std::size_t start = 0;
  c.take(sizeof(kMagic), &start);
  const std::int32_t count = c.pod<std::int32_t>("n_tensors");
  if (count < 0 || count > kMaxTensors) {
    bad_file(f.path, "implausible tensor count " + std::to_string(count));
  }
  f.tensors.reserve(static_cast<std::size_t>(count));
  std::int64_t slab = 0;
  for (std::int32_t t = 0; t < count; ++t) {
    TensorEntry e;
    const std::int32_t name_len = c.pod<std::int32_t>("name_len");
    if (name_len <= 0 || name_len > kMaxNameLen) {
      bad_file(f.path, "implausible name length " + std::to_string(name_len));
    }
    if (!c.take(static_cast<std::size_t>(name_len), &start)) {
      bad_file(f.path, "truncated tensor name");
    }
    e.name.assign(reinterpret_cast<const char*>(f.map + start), static_cast<std::size_t>(name_len));
    e.dtype = c.pod<std::int32_t>("dtype");
    const std::int64_t esize = element_bytes(e.dtype);
    if (esize == 0) {
      bad_file(f.path, "tensor '" + e.name + "' has dtype " + std::to_string(e.dtype) +
                           "; supported: 0 (float32), 1 (float16), 2 (float64)");
    }
    const std::int32_t ndim = c.pod<std::int32_t>("ndim");
    if (ndim < 0 || ndim > kMaxNdim) {
      bad_file(f.path, "implausible ndim " + std::to_string(ndim) + " for '" + e.name + "'");
    }
    std::int64_t numel = 1;
    bool overflow = false;
    for (std::int32_t d = 0; d < ndim; ++d) {
      const std::int64_t v = c.pod<std::int64_t>("dim");
      if (v < 0) bad_file(f.path, "negative dimension in '" + e.name + "'");
      e.dims.push_back(v);
      if (v != 0 && numel > (INT64_MAX / 8) / v) overflow = true;
      numel = overflow ? numel : numel * v;
    }
    e.nbytes = c.pod<std::int64_t>("n_bytes");
    if (overflow) bad_file(f.path, "tensor '" + e.name + "': shape is too large");
    const std::int64_t implied = numel * esize;
    if (e.nbytes != implied) {
      bad_file(f.path, "tensor '" + e.name + "': header says " + std::to_string(e.nbytes) +
                           " bytes but its shape implies " + std::to_string(implied));
    }
    if (!c.take(static_cast<std::size_t>(e.nbytes), &start)) {
      bad_file(f.path, "truncated data for '" + e.name + "'");
    }
    e.file_offset = start;
    slab = (slab + kSlabAlign - 1) / kSlabAlign * kSlabAlign;
    e.slab_offset = slab;
    slab += e.nbytes;
    if (!f.by_name.emplace(e.name, t).second) {
      bad_file(f.path, "duplicate tensor name '" + e.name + "'");
    }
    f.tensors.push_back(std::move(e));
  }
  if (c.pos() != f.size) {
    bad_file(f.path, "unexpected trailing bytes -- writer and reader formats disagree");
  }
  f.slab_bytes = (slab + kSlabAlign - 1) / kSlabAlign * kSlabAlign;
}

const TensorEntry& entry(const eng_engref_s* f, std::int32_t index) {
  ENG_CHECK(index >= 0 && static_cast<std::size_t>(index) < f->tensors.size(),
            "eng_engref_tensor: index " + std::to_string(index) + " out of range for " +
                std::to_string(f->tensors.size()) + " tensors");
  return f->tensors[static_cast<std::size_t>(index)];
}

// Two pinned staging buffers, each guarded by an event recorded after the copy
// that reads it; freed (after a stream sync) when the upload ends.
class Staging {
 public:
  explicit Staging(hipStream_t s) : stream_(s) {}
  // Separate from the constructor so that a failure part-way still runs the
  // destructor over what was allocated.
  void init() {
    for (int i = 0; i < 2; ++i) {
      ENG_HIP_CHECK(hipHostMalloc(&buf_[i], kStageBytes, hipHostMallocDefault));
      ENG_HIP_CHECK(hipEventCreateWithFlags(&done_[i], hipEventDisableTiming));
    }
  }
  ~Staging() {
    (void)hipStreamSynchronize(stream_);
    for (int i = 0; i < 2; ++i) {
      if (done_[i] != nullptr) (void)hipEventDestroy(done_[i]);
      if (buf_[i] != nullptr) (void)hipHostFree(buf_[i]);
    }
  }
  Staging(const Staging&) = delete;
  Staging& operator=(const Staging&) = delete;

  void copy(char* dst, const unsigned char* src, std::size_t bytes) {
    while (bytes > 0) {
      const std::size_t n = bytes < kStageBytes ? bytes : kStageBytes;
      const int i = next_;
      next_ ^= 1;
      if (used_[i]) ENG_HIP_CHECK(hipEventSynchronize(done_[i]));
      std::memcpy(buf_[i], src, n);
      ENG_HIP_CHECK(hipMemcpyAsync(dst, buf_[i], n, hipMemcpyHostToDevice, stream_));
      ENG_HIP_CHECK(hipEventRecord(done_[i], stream_));
      used_[i] = true;
      dst += n;
      src += n;
      bytes -= n;
    }
  }

  void finish() { ENG_HIP_CHECK(hipStreamSynchronize(stream_)); }

 private:
  hipStream_t stream_;
  void* buf_[2] = {nullptr, nullptr};
  hipEvent_t done_[2] = {nullptr, nullptr};
  bool used_[2] = {false, false};
  int next_ = 0;
};

}  // namespace

extern "C" {

int eng_engref_open(const char* path, eng_engref* file) {
  return eng::guarded([&] {
    ENG_CHECK(file != nullptr, "eng_engref_open: file is null");
    *file = nullptr;
    ENG_CHECK(path != nullptr, "eng_engref_open: path is null");
    auto f = std::make_unique<eng_engref_s>();
    f->path = path;
    const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
      const int err = errno;
      eng::raise(ENG_INVALID_ARGUMENT, __FILE__, __LINE__, "open(path)",
                 "cannot open '" + f->path + "': " + std::strerror(err));
    }
    struct stat st {};
    if (fstat(fd, &st) != 0) {
      const int err = errno;
      ::close(fd);
      eng::raise(ENG_INVALID_ARGUMENT, __FILE__, __LINE__, "fstat(path)",
                 "cannot stat '" + f->path + "': " + std::strerror(err));
    }
    f->size = static_cast<std::size_t>(st.st_size);
    if (f->size > 0) {
      void* m = mmap(nullptr, f->size, PROT_READ, MAP_PRIVATE, fd, 0);
      if (m == MAP_FAILED) {
        const int err = errno;
        ::close(fd);
        eng::raise(ENG_INVALID_ARGUMENT, __FILE__, __LINE__, "mmap(path)",
                   "cannot map '" + f->path + "': " + std::strerror(err));
      }
      f->map = static_cast<const unsigned char*>(m);
    }
    ::close(fd);  // the mapping stays valid
    parse(*f);
    *file = f.release();
  });
}

int eng_engref_close(eng_engref file) {
  return eng::guarded([&] { delete file; });
}

int eng_engref_count(eng_engref file, int32_t* count) {
  return eng::guarded([&] {
    ENG_CHECK(file != nullptr, "eng_engref_count: file is null");
    ENG_CHECK(count != nullptr, "eng_engref_count: count is null");
    *count = static_cast<int32_t>(file->tensors.size());
  });
}

int eng_engref_find(eng_engref file, const char* name, int32_t* index) {
  return eng::guarded([&] {
    ENG_CHECK(file != nullptr, "eng_engref_find: file is null");
    ENG_CHECK(name != nullptr, "eng_engref_find: name is null");
    ENG_CHECK(index != nullptr, "eng_engref_find: index is null");
    const auto it = file->by_name.find(name);
    if (it == file->by_name.end()) {
      std::vector<std::string> names;
      for (const auto& t : file->tensors) names.push_back(t.name);
      std::sort(names.begin(), names.end());
      std::string msg = "engref tensor '" + std::string(name) + "' not found. Available:";
      for (const auto& n : names) msg += " " + n;
      eng::raise(ENG_INVALID_ARGUMENT, __FILE__, __LINE__, "name is present", msg);
    }
    *index = it->second;
  });
}

int eng_engref_tensor(eng_engref file, int32_t index, const char** name, int32_t* dtype,
                      int32_t* ndim, const int64_t** dims, int64_t* nbytes,
                      const void** host_data, int64_t* slab_offset) {
  return eng::guarded([&] {
    ENG_CHECK(file != nullptr, "eng_engref_tensor: file is null");
    const TensorEntry& e = entry(file, index);
    if (name != nullptr) *name = e.name.c_str();
    if (dtype != nullptr) *dtype = e.dtype;
    if (ndim != nullptr) *ndim = static_cast<int32_t>(e.dims.size());
    if (dims != nullptr) *dims = e.dims.data();
    if (nbytes != nullptr) *nbytes = e.nbytes;
    if (host_data != nullptr) *host_data = file->map + e.file_offset;
    if (slab_offset != nullptr) *slab_offset = e.slab_offset;
  });
}

int eng_engref_slab_bytes(eng_engref file, int64_t* bytes) {
  return eng::guarded([&] {
    ENG_CHECK(file != nullptr, "eng_engref_slab_bytes: file is null");
    ENG_CHECK(bytes != nullptr, "eng_engref_slab_bytes: bytes is null");
    *bytes = file->slab_bytes;
  });
}

int eng_engref_upload(eng_engref file, void* slab, int64_t capacity, eng_stream stream) {
  return eng::guarded([&] {
    ENG_CHECK(file != nullptr, "eng_engref_upload: file is null");
    ENG_CHECK(capacity >= 0, "eng_engref_upload: capacity must be non-negative");
    ENG_CHECK(capacity >= file->slab_bytes,
              "eng_engref_upload: slab capacity " + std::to_string(capacity) + " < " +
                  std::to_string(file->slab_bytes) + " bytes needed");
    if (file->slab_bytes == 0) return;
    ENG_CHECK(slab != nullptr, "eng_engref_upload: slab is null");
    ENG_CHECK(eng::aligned_to(slab, kSlabAlign), "eng_engref_upload: slab must be 256-byte aligned");
    madvise(const_cast<unsigned char*>(file->map), file->size, MADV_SEQUENTIAL);
    Staging staging(eng::as_stream(stream));
    staging.init();
    char* base = static_cast<char*>(slab);
    for (const auto& e : file->tensors) {
      staging.copy(base + e.slab_offset, file->map + e.file_offset, static_cast<std::size_t>(e.nbytes));
    }
    staging.finish();
  });
}

}  // extern "C"
