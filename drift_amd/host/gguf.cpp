// The GGUF reader of the C++ host (formats/Gguf.scala), with the reference's
// checks and messages.
#include "gguf.hpp"

#include <fcntl.h>
#include <hip/hip_runtime_api.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <sstream>

namespace drift::gguf {

namespace {

// DType.all's GGUF types (tensor/DType.scala:168-193 and the quant objects)
const GgmlType kTypes[] = {
    {"F32", 0, 1, 4},        {"F16", 1, 1, 2},           {"BF16", 30, 1, 2},       {"I8", 24, 1, 1},
    {"I32", 26, 1, 4},       {"I64", 27, 1, 8},          {"Q4_0", 2, 32, 18},      {"Q4_1", 3, 32, 20},
    {"Q5_0", 6, 32, 22},     {"Q5_1", 7, 32, 24},        {"Q8_0", 8, 32, 34},      {"Q2_K", 10, 256, 84},
    {"Q3_K", 11, 256, 110},  {"Q4_K", 12, 256, 144},     {"Q5_K", 13, 256, 176},   {"Q6_K", 14, 256, 210},
    {"IQ4_NL", 20, 32, 18},  {"IQ4_XS", 23, 256, 136},   {"Q4_0_ROCMFP4", 100, 32, 18},
    {"Q4_0_ROCMFP4_FAST", 101, 32, 17}};

// GGML's type ids the runner does not decode, named for the error
// (DType.scala:199-216)
const std::map<int, const char*> kUnsupported = {
    {9, "Q8_1"},    {15, "Q8_K"},    {16, "IQ2_XXS"}, {17, "IQ2_XS"}, {18, "IQ3_XXS"}, {19, "IQ1_S"}, {21, "IQ3_S"},
    {22, "IQ2_S"},  {25, "I16"},     {28, "F64"},     {29, "IQ1_M"},  {34, "TQ1_0"},   {35, "TQ2_0"}, {39, "MXFP4"}};

constexpr int64_t kDefaultAlignment = 32;
constexpr int64_t kRocmSampledBlocks = 4096;  // RocmFp4.scala:41-42

template <typename... Parts>
std::string text(const Parts&... parts) {
  std::ostringstream s;
  (s << ... << parts);
  return s.str();
}

std::string list(const std::vector<int64_t>& dims) {
  std::string s = "[";
  for (size_t i = 0; i < dims.size(); ++i) s += (i ? ", " : "") + std::to_string(dims[i]);
  return s + "]";
}

std::string show(const Value& v) {
  switch (v.kind) {
    case Value::Integer: return std::to_string(v.integer);
    case Value::Real: return text(v.real);
    case Value::Boolean: return v.flag ? "true" : "false";
    case Value::Text: return v.text;
    case Value::Array: return text("an array of ", v.items.size());
  }
  return "?";
}

}  // namespace

int64_t GgmlType::byteSize(int64_t elements) const {
  if (elements % values != 0)
    throw FormatError(text(elements, " elements are not whole ", name, " blocks of ", values));
  int64_t size = 0;
  if (__builtin_mul_overflow(elements / values, (int64_t)bytes, &size))
    throw FormatError(text(elements, " ", name, " elements do not fit 2^63 bytes"));
  return size;
}

const GgmlType* typeOf(int id, std::string& reason) {
  for (const GgmlType& t : kTypes)
    if (t.id == id) return &t;
  const auto named = kUnsupported.find(id);
  reason = named == kUnsupported.end() ? text("unknown GGML type id ", id)
                                       : text("GGML type ", named->second, " is not supported yet");
  return nullptr;
}

// The element count of a shape, refused where it does not fit an int64 (the
// dimensions of a crafted file can multiply past it).
static int64_t elementCount(const std::string& name, const std::vector<int64_t>& shape) {
  int64_t elements = 1;
  for (int64_t d : shape)
    if (__builtin_mul_overflow(elements, d, &elements))
      throw FormatError(text(name, " of ", list(shape), " has more than 2^63 elements"));
  return elements;
}

int64_t StoredTensor::byteSize() const { return type->byteSize(elementCount(name, shape)); }

// ---------------------------------------------------------------- reading

class Reader {
 public:
  Reader(const uint8_t* b, size_t size, std::string source) : b_(b), size_(size), source_(std::move(source)) {}

  [[noreturn]] void fail(const std::string& message) const { throw FormatError(source_ + ": " + message); }

  void need(int64_t n) const {
    if (n < 0 || at_ + n > (int64_t)size_) fail(text("truncated at byte ", at_, " (needs ", n, " more)"));
  }

  template <typename T>
  T take() {
    need((int64_t)sizeof(T));
    T v;
    std::memcpy(&v, b_ + at_, sizeof(T));
    at_ += (int64_t)sizeof(T);
    return v;
  }

  // a count or a length: a u64 that must fit what follows it
  int64_t count(const std::string& what) {
    const int64_t v = take<int64_t>();
    if (v < 0 || v > (int64_t)size_) fail(text(what, " of ", v, " is not plausible"));
    return v;
  }

  std::string string() {
    const int64_t n = count("string length");
    need(n);
    std::string s(reinterpret_cast<const char*>(b_ + at_), (size_t)n);
    at_ += n;
    return s;
  }

  Value value(uint32_t kind) {
    Value v;
    switch (kind) {
      case 0: v.integer = take<uint8_t>(); break;
      case 1: v.integer = take<int8_t>(); break;
      case 2: v.integer = take<uint16_t>(); break;
      case 3: v.integer = take<int16_t>(); break;
      case 4: v.integer = take<uint32_t>(); break;
      case 5: v.integer = take<int32_t>(); break;
      case 10: {
        const uint64_t u = take<uint64_t>();
        v.integer = (int64_t)u;
        v.fits = u <= (uint64_t)INT64_MAX;
        break;
      }
      case 11: v.integer = take<int64_t>(); break;
      case 6: v.kind = Value::Real; v.real = take<float>(); break;
      case 12: v.kind = Value::Real; v.real = take<double>(); break;
      case 7: v.kind = Value::Boolean; v.flag = take<uint8_t>() != 0; break;
      case 8: v.kind = Value::Text; v.text = string(); break;
      case 9: {
        v.kind = Value::Array;
        const uint32_t element = take<uint32_t>();
        const int64_t n = count("array length");
        for (int64_t i = 0; i < n; ++i) v.items.push_back(value(element));
        break;
      }
      default: fail(text("unknown metadata value type ", kind));
    }
    return v;
  }

  void read(File& f) {
    need(8);
    if (std::memcmp(b_, "GGUF", 4) != 0) fail("not a GGUF file");
    at_ = 4;
    const uint32_t version = take<uint32_t>();
    if (version != 2 && version != 3)
      fail(version > 0xFFFF ? std::string("big-endian GGUF is not supported")
                            : text("GGUF version ", version, " is not supported"));
    f.version_ = (int)version;
    const int64_t tensor_count = count("tensor count");
    const int64_t metadata_count = count("metadata count");
    for (int64_t i = 0; i < metadata_count; ++i) {
      std::string key = string();
      const uint32_t kind = take<uint32_t>();
      f.metadata_[key] = value(kind);
    }
    const auto found = f.metadata_.find("general.alignment");
    f.alignment_ = kDefaultAlignment;
    if (found != f.metadata_.end()) {
      const Value& a = found->second;
      if (a.kind != Value::Integer || !a.fits || a.integer <= 0 || (a.integer & (a.integer - 1)) != 0)
        fail(text("general.alignment is ", show(a)));
      f.alignment_ = a.integer;
    }
    struct Info {
      std::string name;
      std::vector<int64_t> dims;
      uint32_t type;
      int64_t offset;
    };
    std::vector<Info> infos;
    for (int64_t i = 0; i < tensor_count; ++i) {
      Info info;
      info.name = string();
      const uint32_t rank = take<uint32_t>();
      if (rank > 8) fail(text(info.name, " has ", rank, " dimensions"));
      for (uint32_t d = 0; d < rank; ++d) info.dims.push_back(count(info.name + " dimension"));
      info.type = take<uint32_t>();
      info.offset = take<int64_t>();
      // an offset before the data section would place the tensor over the
      // header (the reference's bounds-checked slice refuses it when read)
      // (printed as it is: negating INT64_MIN would overflow)
      if (info.offset < 0) fail(text(info.name, " starts at offset ", info.offset, ", before the data section"));
      infos.push_back(std::move(info));
    }
    const int64_t alignment = f.alignment_;
    const int64_t data_start = (at_ + alignment - 1) / alignment * alignment;
    const int64_t data_bytes = (int64_t)size_ - data_start;
    if (data_bytes < 0) fail("truncated before the data section");
    std::map<std::string, StoredTensor> described;
    for (const Info& info : infos) {
      std::string reason;
      const GgmlType* t = typeOf((int)info.type, reason);
      if (!t) {
        f.unsupported_[info.name] = reason;
        continue;
      }
      if (!info.dims.empty() && info.dims[0] % t->values != 0)
        fail(text(info.name, ": rows of ", info.dims[0], " are not whole ", t->name, " blocks"));
      if (info.offset % alignment != 0) fail(text(info.name, " is not aligned to ", alignment));
      // refused before data_start + offset is formed, which an offset near
      // 2^63 would overflow
      if (info.offset > data_bytes) fail(info.name + " runs past the end of the file");
      StoredTensor tensor{info.name, t, std::vector<int64_t>(info.dims.rbegin(), info.dims.rend()),
                          data_start + info.offset};
      int64_t size = 0;
      try {
        size = tensor.byteSize();
      } catch (const FormatError& e) {
        fail(e.what());
      }
      if (size > data_bytes - info.offset) fail(info.name + " runs past the end of the file");
      described[info.name] = tensor;
    }
    // Gguf.checkSpans (Gguf.scala:262-285): each tensor's byte size and the
    // room to the next tensor agree up to the alignment padding
    std::vector<const Info*> by_offset;
    for (const Info& info : infos) by_offset.push_back(&info);
    std::stable_sort(by_offset.begin(), by_offset.end(),
                     [](const Info* a, const Info* b) { return a->offset < b->offset; });
    for (size_t i = 0; i < by_offset.size(); ++i) {
      const auto t = described.find(by_offset[i]->name);
      if (t == described.end()) continue;
      const int64_t end = i + 1 < by_offset.size() ? by_offset[i + 1]->offset : data_bytes;
      const int64_t room = end - by_offset[i]->offset, size = t->second.byteSize();
      if (room < size || room - size >= alignment)
        fail(text(t->first, " is ", t->second.type->name, " ", list(t->second.shape), ", ", size,
                  " bytes, but the file gives it ", room));
    }
    for (const auto& [name, t] : described) rejects(t);
    f.tensors_ = std::move(described);
  }

  // RocmFp4's check that a tensor's scale bytes are finite E4M3 codes
  void rejects(const StoredTensor& t) const {
    const std::string type = t.type->name;
    if (type.rfind("Q4_0_ROCMFP4", 0) != 0) return;
    const bool fast = type == "Q4_0_ROCMFP4_FAST";
    const int offsets[2] = {16, 17};
    const int per_block = fast ? 1 : 2;
    const int64_t blocks = std::min(t.byteSize() / t.type->bytes, kRocmSampledBlocks);
    for (int64_t block = 0; block < blocks; ++block)
      for (int which = 0; which < per_block; ++which) {
        const int64_t where = block * t.type->bytes + offsets[which];
        const uint8_t scale = b_[t.fileOffset + where];
        if (scale > 0x7E) {
          char hex[8];
          std::snprintf(hex, sizeof hex, "0x%02x", scale);
          fail(text(t.name, ": scale byte ", hex, " at byte ", where, " is not a finite unsigned E4M3, so this is not ",
                    type));
        }
      }
  }

 private:
  const uint8_t* b_;
  size_t size_;
  std::string source_;
  int64_t at_ = 0;
};

// ---------------------------------------------------------------- the file

File File::open(const std::string& path) {
  const int fd = ::open(path.c_str(), O_RDONLY);
  if (fd < 0) throw FormatError(path + ": cannot be opened");
  struct stat st;
  if (fstat(fd, &st) != 0) {
    ::close(fd);
    throw FormatError(path + ": cannot be opened");
  }
  const size_t size = (size_t)st.st_size;
  if (size == 0) {
    ::close(fd);
    throw FormatError(path + ": truncated at byte 0 (needs 8 more)");
  }
  void* map = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (map == MAP_FAILED) throw FormatError(path + ": cannot be mapped");
  File f;
  f.source_ = path;
  f.data_ = static_cast<const uint8_t*>(map);
  f.size_ = size;
  Reader(f.data_, size, path).read(f);  // a refusal unmaps through ~File
  return f;
}

File::~File() {
  if (data_) munmap(const_cast<uint8_t*>(data_), size_);
}

File::File(File&& other) noexcept
    : source_(std::move(other.source_)),
      version_(other.version_),
      alignment_(other.alignment_),
      metadata_(std::move(other.metadata_)),
      tensors_(std::move(other.tensors_)),
      unsupported_(std::move(other.unsupported_)),
      data_(other.data_),
      size_(other.size_) {
  other.data_ = nullptr;
  other.size_ = 0;
}

namespace {
const Value& lookup(const std::map<std::string, Value>& m, const std::string& source, const std::string& key) {
  const auto v = m.find(key);
  if (v == m.end()) throw FormatError(source + " has no " + key);
  return v->second;
}
}  // namespace

int64_t File::longValue(const std::string& key) const {
  const Value& v = lookup(metadata_, source_, key);
  if (v.kind != Value::Integer || !v.fits) throw FormatError(source_ + ": " + key + " is " + show(v));
  return v.integer;
}

double File::doubleValue(const std::string& key) const {
  const Value& v = lookup(metadata_, source_, key);
  if (v.kind == Value::Integer) return (double)v.integer;
  if (v.kind != Value::Real) throw FormatError(source_ + ": " + key + " is " + show(v));
  return v.real;
}

std::string File::stringValue(const std::string& key) const {
  const Value& v = lookup(metadata_, source_, key);
  if (v.kind != Value::Text) throw FormatError(source_ + ": " + key + " is " + show(v));
  return v.text;
}

bool File::booleanValue(const std::string& key) const {
  const Value& v = lookup(metadata_, source_, key);
  if (v.kind != Value::Boolean) throw FormatError(source_ + ": " + key + " is " + show(v));
  return v.flag;
}

std::vector<std::string> File::strings(const std::string& key) const {
  const Value& v = lookup(metadata_, source_, key);
  std::vector<std::string> out;
  if (v.kind == Value::Array)
    for (const Value& item : v.items) {
      if (item.kind != Value::Text) throw FormatError(source_ + ": " + key + " is " + show(v));
      out.push_back(item.text);
    }
  else
    throw FormatError(source_ + ": " + key + " is " + show(v));
  return out;
}

const StoredTensor& File::operator[](const std::string& name) const {
  const auto t = tensors_.find(name);
  if (t != tensors_.end()) return t->second;
  const auto u = unsupported_.find(name);
  throw std::out_of_range(u != unsupported_.end() ? name + ": " + u->second : "no tensor " + name);
}

const uint8_t* File::bytes(const std::string& name) const { return data_ + (*this)[name].fileOffset; }

DeviceTable File::table(const std::string& name) const {
  const StoredTensor& t = (*this)[name];
  if (t.shape.size() != 2) throw FormatError(text(name, " is ", list(t.shape), ", not a table"));
  const StorageType* storage = nullptr;
  for (const StorageType& s : StorageType::all())
    if (std::string(s.name) == t.type->name) storage = &s;
  if (!storage) throw FormatError(text(name, ": ", t.type->name, " tables have no gather kernel"));
  const int64_t bytes = t.byteSize();
  void* memory = nullptr;
  hipError_t status = hipMalloc(&memory, (size_t)std::max<int64_t>(bytes, 16));
  if (status == hipSuccess) status = hipMemcpy(memory, data_ + t.fileOffset, (size_t)bytes, hipMemcpyHostToDevice);
  if (status != hipSuccess) {
    if (memory) (void)hipFree(memory);
    throw HipException("hipMemcpy", (int)status, hipGetErrorString(status));
  }
  const int64_t rows = t.shape[0], cols = t.shape[1];
  return DeviceTable(StoredTable{Tensor{DType::U8, {rows, rows ? bytes / rows : 0}, memory}, storage, cols}, memory);
}

DeviceTable::~DeviceTable() {
  if (memory_) (void)hipFree(memory_);
}

DeviceTable::DeviceTable(DeviceTable&& other) noexcept : table_(std::move(other.table_)), memory_(other.memory_) {
  other.memory_ = nullptr;
}

}  // namespace drift::gguf
