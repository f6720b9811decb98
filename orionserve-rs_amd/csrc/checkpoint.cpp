// Safetensors reader: file mapping and header parsing (format: an 8-byte
// little-endian header length N, N bytes of JSON mapping each tensor name to
// {"dtype", "shape", "data_offsets": [begin, end]} relative to the byte
// buffer that follows the header, plus an optional "__metadata__" object).
#include "checkpoint.hpp"

#include <dirent.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>

#include "../../include/orion_hip.h"

namespace orion {

namespace {

// A minimal JSON reader for the header: objects, arrays, strings, integers
// and the literals; anything else is a malformed header.
class JsonReader {
 public:
  JsonReader(const char* p, size_t n) : p_(p), end_(p + n) {}

  bool ok() const { return err_.empty(); }
  const std::string& error() const { return err_; }

  void ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
  }
  bool peek(char c) {
    ws();
    return p_ < end_ && *p_ == c;
  }
  bool expect(char c) {
    ws();
    if (p_ < end_ && *p_ == c) {
      ++p_;
      return true;
    }
    return fail(std::string("expected '") + c + "'");
  }
  bool fail(const std::string& what) {
    if (err_.empty()) err_ = what + " at header byte " + std::to_string(pos());
    return false;
  }
  size_t pos() const { return (size_t)(p_ - begin_ + offset_); }

  bool string(std::string* out) {
    if (!expect('"')) return false;
    out->clear();
    while (p_ < end_ && *p_ != '"') {
      char c = *p_++;
      if (c == '\\') {
        if (p_ >= end_) return fail("unterminated escape");
        const char e = *p_++;
        switch (e) {
          case '"': case '\\': case '/': out->push_back(e); break;
          case 'b': out->push_back('\b'); break;
          case 'f': out->push_back('\f'); break;
          case 'n': out->push_back('\n'); break;
          case 'r': out->push_back('\r'); break;
          case 't': out->push_back('\t'); break;
          case 'u': {
            if (end_ - p_ < 4) return fail("short \\u escape");
            unsigned v = 0;
            for (int i = 0; i < 4; ++i) {
              const char h = *p_++;
              v <<= 4;
              if (h >= '0' && h <= '9') v |= (unsigned)(h - '0');
              else if (h >= 'a' && h <= 'f') v |= (unsigned)(h - 'a' + 10);
              else if (h >= 'A' && h <= 'F') v |= (unsigned)(h - 'A' + 10);
              else return fail("bad \\u escape");
            }
            // UTF-8 encode (surrogate pairs are not needed for tensor names
            // in practice; a lone surrogate is kept as its code unit)
            if (v < 0x80) {
              out->push_back((char)v);
            } else if (v < 0x800) {
              out->push_back((char)(0xC0 | (v >> 6)));
              out->push_back((char)(0x80 | (v & 0x3F)));
            } else {
              out->push_back((char)(0xE0 | (v >> 12)));
              out->push_back((char)(0x80 | ((v >> 6) & 0x3F)));
              out->push_back((char)(0x80 | (v & 0x3F)));
            }
            break;
          }
          default: return fail("bad escape");
        }
      } else {
        out->push_back(c);
      }
    }
    if (p_ >= end_) return fail("unterminated string");
    ++p_;
    return true;
  }

  bool integer(int64_t* out) {
    ws();
    const char* s = p_;
    if (p_ < end_ && *p_ == '-') ++p_;
    if (p_ >= end_ || *p_ < '0' || *p_ > '9') return fail("expected an integer");
    uint64_t v = 0;
    while (p_ < end_ && *p_ >= '0' && *p_ <= '9') {
      if (v > (uint64_t)INT64_MAX / 10) return fail("integer out of range");
      v = v * 10 + (uint64_t)(*p_++ - '0');
    }
    if (p_ < end_ && (*p_ == '.' || *p_ == 'e' || *p_ == 'E')) return fail("expected an integer");
    *out = (*s == '-') ? -(int64_t)v : (int64_t)v;
    return true;
  }

  bool int_array(std::vector<int64_t>* out) {
    out->clear();
    if (!expect('[')) return false;
    if (peek(']')) return expect(']');
    while (true) {
      int64_t v;
      if (!integer(&v)) return false;
      out->push_back(v);
      if (peek(',')) {
        expect(',');
        continue;
      }
      return expect(']');
    }
  }

  // Skips any JSON value (for "__metadata__" and unknown keys).
  bool skip(int depth = 0) {
    if (depth > 64) return fail("nesting too deep");
    ws();
    if (p_ >= end_) return fail("unexpected end");
    const char c = *p_;
    if (c == '"') {
      std::string tmp;
      return string(&tmp);
    }
    if (c == '{' || c == '[') {
      const char close = c == '{' ? '}' : ']';
      ++p_;
      if (peek(close)) return expect(close);
      while (true) {
        if (c == '{') {
          std::string k;
          if (!string(&k) || !expect(':')) return false;
        }
        if (!skip(depth + 1)) return false;
        if (peek(',')) {
          expect(',');
          continue;
        }
        return expect(close);
      }
    }
    for (const char* lit : {"true", "false", "null"}) {
      const size_t n = strlen(lit);
      if ((size_t)(end_ - p_) >= n && memcmp(p_, lit, n) == 0) {
        p_ += n;
        return true;
      }
    }
    if (c == '-' || (c >= '0' && c <= '9')) {
      ++p_;
      while (p_ < end_ && (strchr("0123456789+-.eE", *p_) != nullptr)) ++p_;
      return true;
    }
    return fail("unexpected character");
  }

  bool at_end() {
    ws();
    return p_ == end_;
  }

 private:
  const char* p_;
  const char* end_;
  const char* begin_ = p_;
  size_t offset_ = 8;  // header JSON starts after the 8-byte length
  std::string err_;
};

int dtype_code(const std::string& s, size_t* elem) {
  if (s == "F32") {
    *elem = 4;
    return ORION_DTYPE_F32;
  }
  if (s == "F16") {
    *elem = 2;
    return ORION_DTYPE_F16;
  }
  if (s == "BF16") {
    *elem = 2;
    return ORION_DTYPE_BF16;
  }
  // Other safetensors dtypes: sizes for the offset check only.
  static const std::pair<const char*, size_t> other[] = {
      {"F64", 8}, {"I64", 8}, {"U64", 8}, {"I32", 4}, {"U32", 4}, {"I16", 2}, {"U16", 2},
      {"I8", 1},  {"U8", 1},  {"BOOL", 1}, {"F8_E4M3", 1}, {"F8_E5M2", 1}};
  for (const auto& o : other)
    if (s == o.first) {
      *elem = o.second;
      return -1;
    }
  *elem = 0;
  return -1;
}

// Parses one file's header into `out` (name -> tensor, data pointers into
// the mapping).  Returns an empty string or the reason the file is malformed.
std::string parse_header(const char* base, size_t size,
                         std::vector<CheckpointTensor>* out) {
  if (size < 8) return "file shorter than the 8-byte header length";
  uint64_t n = 0;
  for (int i = 7; i >= 0; --i) n = (n << 8) | (uint8_t)base[i];
  if (n > size - 8) return "header length " + std::to_string(n) + " exceeds the file";
  const char* data = base + 8 + n;
  const size_t data_size = size - 8 - (size_t)n;
  JsonReader r(base + 8, (size_t)n);
  if (!r.expect('{')) return r.error();
  std::vector<std::pair<int64_t, int64_t>> ranges;
  if (!r.peek('}')) {
    while (true) {
      std::string key;
      if (!r.string(&key) || !r.expect(':')) return r.error();
      if (key == "__metadata__") {
        if (!r.skip()) return r.error();
      } else {
        CheckpointTensor t;
        t.name = key;
        std::vector<int64_t> offs;
        bool have_dtype = false, have_shape = false, have_offs = false;
        if (!r.expect('{')) return r.error();
        if (!r.peek('}')) {
          while (true) {
            std::string f;
            if (!r.string(&f) || !r.expect(':')) return r.error();
            if (f == "dtype") {
              if (!r.string(&t.dtype_name)) return r.error();
              have_dtype = true;
            } else if (f == "shape") {
              if (!r.int_array(&t.shape)) return r.error();
              have_shape = true;
            } else if (f == "data_offsets") {
              if (!r.int_array(&offs)) return r.error();
              have_offs = true;
            } else if (!r.skip()) {
              return r.error();
            }
            if (r.peek(',')) {
              r.expect(',');
              continue;
            }
            if (!r.expect('}')) return r.error();
            break;
          }
        } else {
          r.expect('}');
        }
        if (!have_dtype || !have_shape || !have_offs || offs.size() != 2)
          return "tensor `" + key + "` lacks dtype, shape or data_offsets";
        size_t elem = 0;
        t.dtype = dtype_code(t.dtype_name, &elem);
        if (elem == 0) return "tensor `" + key + "` has unknown dtype " + t.dtype_name;
        int64_t count = 1;
        for (int64_t d : t.shape) {
          if (d < 0 || (d > 0 && count > INT64_MAX / d))
            return "tensor `" + key + "` has an invalid shape";
          count *= d;
        }
        if (offs[0] < 0 || offs[1] < offs[0] || (uint64_t)offs[1] > data_size)
          return "tensor `" + key + "` data_offsets fall outside the file";
        // count * elem computed only once it cannot wrap (count <= data_size)
        if ((uint64_t)count > data_size / elem ||
            (uint64_t)(offs[1] - offs[0]) != (uint64_t)count * elem)
          return "tensor `" + key + "` data_offsets do not match its shape and dtype";
        t.data = data + offs[0];
        t.bytes = (size_t)(offs[1] - offs[0]);
        ranges.push_back({offs[0], offs[1]});
        out->push_back(std::move(t));
      }
      if (r.peek(',')) {
        r.expect(',');
        continue;
      }
      if (!r.expect('}')) return r.error();
      break;
    }
  } else {
    r.expect('}');
  }
  if (!r.at_end()) return "trailing bytes after the header object";
  std::sort(ranges.begin(), ranges.end());
  for (size_t i = 1; i < ranges.size(); ++i)
    if (ranges[i].first < ranges[i - 1].second) return "tensor data ranges overlap";
  return "";
}

}  // namespace

std::unique_ptr<Checkpoint> Checkpoint::open(const std::string& dir, Error* kind,
                                             std::string* err) {
  *kind = Error::kNone;
  struct stat st {};
  if (stat(dir.c_str(), &st) != 0) {
    *kind = Error::kPathNotFound;
    *err = "path not found: " + dir;
    return nullptr;
  }
  DIR* d = opendir(dir.c_str());
  if (!d) {
    *kind = Error::kIo;
    *err = "cannot read directory " + dir + ": " + strerror(errno);
    return nullptr;
  }
  std::vector<std::string> paths;
  while (dirent* e = readdir(d)) {
    const std::string name = e->d_name;
    const std::string ext = ".safetensors";
    if (name.size() > ext.size() && name.compare(name.size() - ext.size(), ext.size(), ext) == 0)
      paths.push_back(dir + "/" + name);
  }
  closedir(d);
  // Sorted, so a tensor name present in two files always resolves the same way.
  std::sort(paths.begin(), paths.end());
  if (paths.empty()) {
    *kind = Error::kMissingFile;
    *err = "missing file: " + dir + "/*.safetensors";
    return nullptr;
  }
  std::unique_ptr<Checkpoint> ck(new Checkpoint());
  for (const std::string& path : paths) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) {
      *kind = Error::kIo;
      *err = "cannot open " + path + ": " + strerror(errno);
      return nullptr;
    }
    struct stat fs {};
    if (fstat(fd, &fs) != 0) {
      *kind = Error::kIo;
      *err = "cannot stat " + path + ": " + strerror(errno);
      ::close(fd);
      return nullptr;
    }
    Map m;
    m.path = path;
    m.size = (size_t)fs.st_size;
    if (m.size > 0) {
      m.base = mmap(nullptr, m.size, PROT_READ, MAP_PRIVATE, fd, 0);
      if (m.base == MAP_FAILED) {
        m.base = nullptr;
        *kind = Error::kIo;
        *err = "cannot map " + path + ": " + strerror(errno);
        ::close(fd);
        return nullptr;
      }
    }
    ::close(fd);  // the mapping stays valid
    ck->maps_.push_back(m);
    std::vector<CheckpointTensor> tensors;
    const std::string why = parse_header(static_cast<const char*>(m.base), m.size, &tensors);
    if (!why.empty()) {
      *kind = Error::kMalformed;
      *err = "malformed " + path + ": " + why;
      return nullptr;
    }
    for (auto& t : tensors) ck->index_.emplace(t.name, std::move(t));  // first file wins
  }
  for (const auto& kv : ck->index_) ck->names_.push_back(kv.first);
  return ck;
}

Checkpoint::~Checkpoint() {
  for (const Map& m : maps_)
    if (m.base) munmap(m.base, m.size);
}

const CheckpointTensor* Checkpoint::find(const std::string& name) const {
  const auto it = index_.find(name);
  return it == index_.end() ? nullptr : &it->second;
}

}  // namespace orion
