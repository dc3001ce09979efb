// kanjoos_amd/csrc/knj_gguf.h -- read-only view of a GGUF (version 2/3) file:
// the metadata scalars and the tensor table, over a memory map.  Host code.
//
// Written from the GGUF container format: "GGUF", version, tensor count,
// metadata count; metadata as (string key, u32 type, value); tensor infos as
// (string name, u32 n_dims, u64 dims[n_dims] with dims[0] fastest, u32 ggml
// type, u64 offset); tensor data from the first multiple of
// general.alignment (default 32) after the infos.  Arrays (the tokenizer's
// vocabulary and merges) are skipped: the decode path does not use them.
// Every read is bounds-checked; a malformed file yields an error string.
#pragma once

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdint>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/knj_format.h"

namespace knj {

// A string read from a file, as it may appear in an error message: printable
// ASCII kept, every other byte as \xNN, at most 64 bytes of it.
inline std::string gguf_printable(const std::string& v) {
  static const char* hex = "0123456789abcdef";
  std::string out;
  for (size_t i = 0; i < v.size() && i < 64; ++i) {
    const unsigned char ch = (unsigned char)v[i];
    if (ch >= 0x20 && ch < 0x7f) {
      out += (char)ch;
    } else {
      out += "\\x";
      out += hex[ch >> 4];
      out += hex[ch & 15];
    }
  }
  if (v.size() > 64) out += "...";
  return out;
}

struct GgufScalar {
  enum Kind { kInt, kFloat, kString } kind = kInt;
  int64_t i = 0;
  double f = 0.0;
  std::string s;
};

struct GgufTensor {
  std::string name;
  uint32_t n_dims = 0;
  uint64_t dims[4] = {1, 1, 1, 1};
  uint32_t type = 0;
  uint64_t offset = 0;  // from the start of the data section
  uint64_t bytes = 0;   // ggml row bytes of dims[0] times the other dims
};

class GgufView {
 public:
  GgufView() = default;
  GgufView(const GgufView&) = delete;
  GgufView& operator=(const GgufView&) = delete;
  ~GgufView() { close(); }

  bool open(const char* path) {
    close();
    fd_ = ::open(path, O_RDONLY);
    if (fd_ < 0) return fail(std::string("cannot open ") + path);
    struct stat st {};
    if (fstat(fd_, &st) != 0 || st.st_size < 24) return fail("not a GGUF file (too short)");
    size_ = (size_t)st.st_size;
    map_ = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0);
    if (map_ == MAP_FAILED) {
      map_ = nullptr;
      return fail("mmap failed");
    }
    return parse();
  }

  void close() {
    if (map_) munmap(map_, size_);
    if (fd_ >= 0) ::close(fd_);
    map_ = nullptr;
    fd_ = -1;
  }

  const std::string& error() const { return err_; }
  const uint8_t* data(const GgufTensor& t) const {
    return static_cast<const uint8_t*>(map_) + data_ + t.offset;
  }
  const GgufTensor* find(const std::string& name) const {
    auto it = index_.find(name);
    return it == index_.end() ? nullptr : &tensors_[it->second];
  }
  const GgufScalar* meta(const std::string& key) const {
    auto it = meta_.find(key);
    return it == meta_.end() ? nullptr : &it->second;
  }
  bool meta_int(const std::string& key, int64_t& v) const {
    const GgufScalar* s = meta(key);
    if (!s || s->kind == GgufScalar::kString) return false;
    v = s->kind == GgufScalar::kInt ? s->i : (int64_t)s->f;
    return true;
  }
  bool meta_float(const std::string& key, double& v) const {
    const GgufScalar* s = meta(key);
    if (!s || s->kind == GgufScalar::kString) return false;
    v = s->kind == GgufScalar::kFloat ? s->f : (double)s->i;
    return true;
  }
  std::string meta_string(const std::string& key) const {
    const GgufScalar* s = meta(key);
    return s && s->kind == GgufScalar::kString ? s->s : std::string();
  }

 private:
  bool fail(const std::string& m) {
    err_ = m;
    return false;
  }
  bool need(uint64_t n) {
    if (pos_ > size_ || n > size_ - pos_) return fail("truncated GGUF file");
    return true;
  }
  template <class T>
  bool rd(T& v) {
    if (!need(sizeof(T))) return false;
    std::memcpy(&v, static_cast<const uint8_t*>(map_) + pos_, sizeof(T));
    pos_ += sizeof(T);
    return true;
  }
  bool rd_str(std::string& s) {
    uint64_t n = 0;
    if (!rd(n) || !need(n)) return false;
    s.assign(reinterpret_cast<const char*>(map_) + pos_, (size_t)n);
    pos_ += n;
    return true;
  }
  // one value of `type`; scalars are kept in `out` when it is given
  bool rd_value(uint32_t type, GgufScalar* out, int depth = 0) {
    if (depth > 2) return fail("nested GGUF arrays");
    auto keep_i = [&](int64_t v) {
      if (out) { out->kind = GgufScalar::kInt; out->i = v; }
    };
    auto keep_f = [&](double v) {
      if (out) { out->kind = GgufScalar::kFloat; out->f = v; }
    };
    switch (type) {
      case 0: { uint8_t v; if (!rd(v)) return false; keep_i(v); return true; }
      case 1: { int8_t v; if (!rd(v)) return false; keep_i(v); return true; }
      case 2: { uint16_t v; if (!rd(v)) return false; keep_i(v); return true; }
      case 3: { int16_t v; if (!rd(v)) return false; keep_i(v); return true; }
      case 4: { uint32_t v; if (!rd(v)) return false; keep_i(v); return true; }
      case 5: { int32_t v; if (!rd(v)) return false; keep_i(v); return true; }
      case 6: { float v; if (!rd(v)) return false; keep_f(v); return true; }
      case 7: { uint8_t v; if (!rd(v)) return false; keep_i(v != 0); return true; }
      case 8: {
        std::string s;
        if (!rd_str(s)) return false;
        if (out) { out->kind = GgufScalar::kString; out->s = std::move(s); }
        return true;
      }
      case 9: {
        uint32_t et = 0;
        uint64_t n = 0;
        if (!rd(et) || !rd(n)) return false;
        for (uint64_t i = 0; i < n; ++i)
          if (!rd_value(et, nullptr, depth + 1)) return false;
        return true;
      }
      case 10: { uint64_t v; if (!rd(v)) return false; keep_i((int64_t)v); return true; }
      case 11: { int64_t v; if (!rd(v)) return false; keep_i(v); return true; }
      case 12: { double v; if (!rd(v)) return false; keep_f(v); return true; }
      default: return fail("unknown GGUF value type " + std::to_string(type));
    }
  }

  bool parse() {
    pos_ = 0;
    uint32_t magic = 0, version = 0;
    uint64_t n_tensors = 0, n_kv = 0;
    if (!rd(magic) || magic != 0x46554747u) return fail("not a GGUF file (bad magic)");
    if (!rd(version) || version < 2 || version > 3) return fail("unsupported GGUF version");
    if (!rd(n_tensors) || !rd(n_kv)) return false;
    if (n_tensors > (1u << 20) || n_kv > (1u << 20)) return fail("implausible GGUF counts");
    for (uint64_t i = 0; i < n_kv; ++i) {
      std::string key;
      uint32_t type = 0;
      if (!rd_str(key) || !rd(type)) return false;
      GgufScalar v;
      if (!rd_value(type, &v)) return false;
      if (type != 9) meta_[key] = std::move(v);
    }
    tensors_.resize((size_t)n_tensors);
    for (uint64_t i = 0; i < n_tensors; ++i) {
      GgufTensor& t = tensors_[(size_t)i];
      if (!rd_str(t.name) || !rd(t.n_dims)) return false;
      if (t.n_dims < 1 || t.n_dims > 4) return fail("tensor '" + gguf_printable(t.name) + "': bad rank");
      for (uint32_t d = 0; d < t.n_dims; ++d)
        if (!rd(t.dims[d])) return false;
      if (!rd(t.type) || !rd(t.offset)) return false;
      // sizes of the types this path reads; other types keep bytes = 0 and are
      // refused by the binder only if the path needs them
      if (knj_row_bytes((int)t.type, 256) != 0) {
        if (t.dims[0] % knj_block_weights((int)t.type))
          return fail("tensor '" + gguf_printable(t.name) + "': row not a whole number of blocks");
        t.bytes = knj_row_bytes((int)t.type, t.dims[0]);
        for (uint32_t d = 1; d < t.n_dims; ++d) t.bytes *= t.dims[d];
      }
      index_[t.name] = (size_t)i;
    }
    int64_t align = 32;
    meta_int("general.alignment", align);
    if (align <= 0 || (align & (align - 1))) return fail("bad general.alignment");
    data_ = (pos_ + (uint64_t)align - 1) / (uint64_t)align * (uint64_t)align;
    for (const GgufTensor& t : tensors_)
      if (data_ > size_ || t.offset > size_ - data_ || t.bytes > size_ - data_ - t.offset)
        return fail("tensor '" + gguf_printable(t.name) + "' extends past the end of the file");
    return true;
  }

  int fd_ = -1;
  void* map_ = nullptr;
  size_t size_ = 0;
  uint64_t pos_ = 0, data_ = 0;
  std::string err_;
  std::unordered_map<std::string, GgufScalar> meta_;
  std::vector<GgufTensor> tensors_;
  std::unordered_map<std::string, size_t> index_;
};

}  // namespace knj
