// GGUF container reader: directory parse and raw tensor upload to device memory.
//
// Counterpart of the reference's directory reader tc::gguf::read_directory and
// validate_split_set (native/core/gguf_directory.hpp:199-304; type table :19-26, limits
// :45-50). What is shared with the reference is the interface: the GGUF v2/v3 format, the
// accepted type table, the parser limits, and the error contract (the "gguf_invalid: <reason>"
// strings and which error a malformed file reports first). The reader itself is built
// differently: the leading directory bytes are loaded into memory on demand and decoded from
// there, retained strings live in one arena referenced by offset, duplicates are found through
// a hash index, metadata arrays are skipped with an explicit frame stack, and split sets are
// checked by a per-shard accumulator. Tensor payloads are read with pread() into pinned
// bounce buffers and copied to device memory, so a Q4_K / Q6_K weight arrives in HBM as the raw
// blocks the kernels consume (no host-side decode).
#include "../../include/tc_qlinear.h"

#include <hip/hip_runtime.h>

#include <errno.h>
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <condition_variable>
#include <cstdint>
#include <deque>
#include <memory>
#include <mutex>
#include <thread>
#include <cstring>
#include <numeric>
#include <stdexcept>
#include <string>
#include <string_view>
#include <unordered_map>
#include <unordered_set>
#include <utility>
#include <vector>

namespace {

[[noreturn]] void invalid(const char *reason) { throw std::invalid_argument(std::string("gguf_invalid: ") + reason); }
void expect(bool ok, const char *reason) {
    if (!ok) invalid(reason);
}
uint64_t sum(uint64_t a, uint64_t b) {
    expect(a <= UINT64_MAX - b, "integer addition overflow");
    return a + b;
}
uint64_t product(uint64_t a, uint64_t b) {
    expect(a == 0 || b <= UINT64_MAX / a, "integer multiplication overflow");
    return a * b;
}

// Block geometry of the accepted GGML tensor types (the file format's type table,
// gguf_directory.hpp:21-26): {id, elements per block, bytes per block}.
struct Geometry {
    uint32_t id, elements, bytes;
};
constexpr Geometry kGeometry[] = {{0, 1, 4},    {1, 1, 2},    {2, 32, 18},   {3, 32, 20},   {6, 32, 22}, {7, 32, 24},
                                  {8, 32, 34},  {12, 256, 144}, {13, 256, 176}, {14, 256, 210}, {30, 1, 2}};
const Geometry &geometry_of(uint32_t id) {
    const Geometry *g = std::find_if(std::begin(kGeometry), std::end(kGeometry), [&](const Geometry &x) { return x.id == id; });
    if (g == std::end(kGeometry)) throw std::invalid_argument("gguf_type_unsupported: " + std::to_string(id));
    return *g;
}

// Parser limits (the reference's defaults, gguf_directory.hpp:45-50).
constexpr uint64_t kMaxTensors = 65536, kMaxMetadata = 65536;
constexpr uint64_t kMaxDirectoryBytes = 64ull << 20, kMaxRetainedBytes = 32ull << 20;
constexpr uint64_t kMaxStringBytes = 1ull << 20, kMaxArrayElements = 1ull << 20;
constexpr uint32_t kMaxRank = 4, kMaxArrayDepth = 4;

// GGUF metadata value types: 0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32, 7 bool, 8 string,
// 9 array, 10 u64, 11 i64, 12 f64. Byte width of the scalar ones (0 for string and array).
constexpr uint8_t kWidth[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
constexpr uint32_t kString = 8, kArray = 9, kBool = 7;
uint32_t scalar_width(uint32_t type) {
    if (type > 12 || kWidth[type] == 0) invalid("invalid metadata scalar type");
    return kWidth[type];
}

// The first bytes of the file, loaded on demand (growing by doubling, never past the file size
// or the directory byte limit) and consumed front to back.
class DirectoryBytes {
  public:
    DirectoryBytes(int fd, uint64_t file_bytes) : fd_(fd), file_bytes_(file_bytes) {}
    uint64_t offset() const { return at_; }
    // Bytes left before the end of the file / of the directory limit.
    uint64_t left_in_file() const { return file_bytes_ > at_ ? file_bytes_ - at_ : 0; }
    uint64_t left_in_limit() const { return kMaxDirectoryBytes > at_ ? kMaxDirectoryBytes - at_ : 0; }
    // Consumes `n` bytes and returns where they start in memory (valid until the next call).
    const uint8_t *consume(uint64_t n) {
        expect(at_ <= file_bytes_ && n <= file_bytes_ - at_, "truncated directory");
        expect(at_ <= kMaxDirectoryBytes && n <= kMaxDirectoryBytes - at_, "directory byte limit");
        load_through(at_ + n);
        const uint8_t *p = buf_.data() + at_;
        at_ += n;
        return p;
    }
    template <typename T>
    T scalar() {
        const uint8_t *p = consume(sizeof(T));
        T v = 0;
        for (size_t b = 0; b < sizeof(T); ++b) v |= (T)((T)p[b] << (8 * b));
        return v;
    }
    uint64_t bits(uint32_t width) {  // little-endian unsigned value of `width` bytes
        const uint8_t *p = consume(width);
        uint64_t v = 0;
        for (uint32_t b = 0; b < width; ++b) v |= (uint64_t)p[b] << (8 * b);
        return v;
    }

  private:
    void load_through(uint64_t end) {
        if (end <= buf_.size()) return;
        const uint64_t cap = std::min(file_bytes_, kMaxDirectoryBytes);
        const uint64_t want = std::min(cap, std::max<uint64_t>(end, std::max<uint64_t>(buf_.size() * 2, 1 << 16)));
        const uint64_t have = buf_.size();
        buf_.resize(want);
        for (uint64_t got = have; got < want;) {
            const ssize_t r = ::pread(fd_, buf_.data() + got, want - got, (off_t)got);
            if (r < 0 && errno == EINTR) continue;
            if (r <= 0) {
                buf_.resize(got);
                invalid("directory read failed or source changed");
            }
            got += (uint64_t)r;
        }
    }
    int fd_;
    uint64_t file_bytes_, at_ = 0;
    std::vector<uint8_t> buf_;
};

struct MetaEntry {
    uint32_t key_at, key_len;   // in the arena
    uint32_t type, element_type;
    uint64_t count, bits;       // array: element count; scalar: raw bits
    int64_t as_signed;
    double as_float;
    uint32_t text_at, text_len;  // string value in the arena
};

struct TensorEntry {
    uint32_t name_at, name_len;
    uint32_t type, rank;
    uint64_t dims[kMaxRank];     // GGML order: dims[0] contiguous
    uint64_t elements, bytes, relative, absolute;
};

}  // namespace

struct tc_gguf_file {
    int fd = -1;
    uint64_t file_bytes = 0;
    uint32_t version = 0, alignment = 32;
    uint64_t directory_end = 0, data_offset = 0;
    uint64_t retained = 0;       // bytes this directory retains (records + arena)
    std::string arena;           // every retained string, NUL-terminated, back to back
    std::vector<MetaEntry> meta;
    std::vector<TensorEntry> tensors;
    std::unordered_map<std::string_view, uint32_t> meta_index, tensor_index;  // built after the parse

    std::string_view str(uint32_t at, uint32_t len) const { return std::string_view(arena.data() + at, len); }
    const char *c_str(uint32_t at) const { return arena.data() + at; }
    const MetaEntry *find_meta(std::string_view key) const {
        const auto it = meta_index.find(key);
        return it == meta_index.end() ? nullptr : &meta[it->second];
    }
};

namespace {

// Directory decoder: fills a tc_gguf_file from its DirectoryBytes, enforcing the limits and
// the format's consistency rules in the reference's first-error order.
class DirectoryParser {
  public:
    DirectoryParser(tc_gguf_file &f) : f_(f), in_(f.fd, f.file_bytes) {}

    void run() {
        expect(in_.scalar<uint32_t>() == 0x46554747u, "invalid GGUF magic/endian");
        f_.version = in_.scalar<uint32_t>();
        expect(f_.version == 2 || f_.version == 3, "unsupported GGUF version");
        const uint64_t n_tensors = in_.scalar<uint64_t>(), n_meta = in_.scalar<uint64_t>();
        expect(n_tensors != 0 && n_tensors <= kMaxTensors && n_tensors <= f_.file_bytes / 24, "tensor count limit");
        expect(n_meta <= kMaxMetadata && n_meta <= f_.file_bytes / 12, "metadata count limit");
        // The record arrays are sized up front and count against the retained budget.
        retain(sum(product(n_tensors, sizeof(TensorEntry)), product(n_meta, sizeof(MetaEntry))));
        f_.meta.reserve(n_meta);
        f_.tensors.reserve(n_tensors);
        for (uint64_t i = 0; i < n_meta; ++i) read_metadata();
        apply_alignment();
        seen_.clear();
        for (uint64_t i = 0; i < n_tensors; ++i) read_tensor();
        place_payloads();
        for (uint32_t i = 0; i < f_.meta.size(); ++i)
            f_.meta_index.emplace(f_.str(f_.meta[i].key_at, f_.meta[i].key_len), i);
        for (uint32_t i = 0; i < f_.tensors.size(); ++i)
            f_.tensor_index.emplace(f_.str(f_.tensors[i].name_at, f_.tensors[i].name_len), i);
    }

  private:
    void retain(uint64_t bytes) {
        f_.retained = sum(f_.retained, bytes);
        expect(f_.retained <= kMaxRetainedBytes, "retained metadata limit");
    }

    // A length-prefixed string kept in the arena: returns its arena offset and length.
    std::pair<uint32_t, uint32_t> kept_string() {
        const uint64_t n = in_.scalar<uint64_t>();
        expect(n <= kMaxStringBytes, "string byte limit");
        retain(n + 1);
        expect(n <= in_.left_in_file() && n <= in_.left_in_limit(), "truncated string");
        const uint8_t *p = in_.consume(n);
        const uint32_t at = (uint32_t)f_.arena.size();
        f_.arena.append(reinterpret_cast<const char *>(p), (size_t)n);
        f_.arena.push_back('\0');
        return {at, (uint32_t)n};
    }
    void skipped_string() {
        const uint64_t n = in_.scalar<uint64_t>();
        expect(n <= kMaxStringBytes, "string byte limit");
        in_.consume(n);
    }

    // Duplicate detection over arena strings: hash -> indices of the entries with that hash.
    bool first_occurrence(uint32_t at, uint32_t len) {
        const std::string_view s = f_.str(at, len);
        auto &bucket = seen_[std::hash<std::string_view>{}(s)];
        for (const auto &[other_at, other_len] : bucket)
            if (f_.str(other_at, other_len) == s) return false;
        bucket.emplace_back(at, len);
        return true;
    }

    // Array payload: element type, count, then the elements. Fixed-width scalars (bool excepted,
    // whose bytes are checked) are skipped in one step; strings, booleans and nested arrays one
    // element at a time, nested arrays through an explicit stack of frames.
    void skip_array(uint32_t depth, MetaEntry *entry) {
        struct Frame {
            uint32_t element;
            uint64_t left;
        };
        Frame stack[kMaxArrayDepth + 1];
        int top = -1;
        auto open = [&](uint32_t level, MetaEntry *e) {
            expect(level < kMaxArrayDepth, "nested array depth limit");
            const uint32_t element = in_.scalar<uint32_t>();
            const uint64_t count = in_.scalar<uint64_t>();
            expect(count <= kMaxArrayElements, "array element limit");
            expect(element <= 12, "invalid array element type");
            if (e) {
                e->element_type = element;
                e->count = count;
            }
            if (element != kString && element != kArray && element != kBool) {
                in_.consume(product(count, kWidth[element]));
                return;
            }
            stack[++top] = Frame{element, count};
        };
        open(depth, entry);
        while (top >= 0) {
            Frame &fr = stack[top];
            if (fr.left == 0) {
                --top;
                continue;
            }
            --fr.left;
            if (fr.element == kString) skipped_string();
            else if (fr.element == kBool) expect(in_.bits(1) <= 1, "invalid boolean");
            else open(depth + (uint32_t)top + 1, nullptr);
        }
    }

    void read_value(MetaEntry &e) {
        if (e.type == kString) {
            std::tie(e.text_at, e.text_len) = kept_string();
            return;
        }
        if (e.type == kArray) {
            skip_array(0, &e);
            return;
        }
        const uint32_t width = scalar_width(e.type);
        e.bits = in_.bits(width);
        if (e.type == kBool) expect(e.bits <= 1, "invalid boolean");
        const bool is_signed = e.type == 1 || e.type == 3 || e.type == 5 || e.type == 11;
        if (is_signed) {
            const unsigned shift = 64 - 8 * width;  // sign-extend the low `width` bytes
            e.as_signed = (int64_t)(e.bits << shift) >> shift;
        }
        if (e.type == 6) {
            float v;
            const uint32_t b = (uint32_t)e.bits;
            std::memcpy(&v, &b, sizeof v);
            e.as_float = v;
        } else if (e.type == 12) {
            std::memcpy(&e.as_float, &e.bits, sizeof e.as_float);
        }
    }

    void read_metadata() {
        MetaEntry e{};
        std::tie(e.key_at, e.key_len) = kept_string();
        const std::string_view key = f_.str(e.key_at, e.key_len);
        expect(!key.empty() && key.find('\0') == std::string_view::npos, "invalid metadata key");
        expect(first_occurrence(e.key_at, e.key_len), "duplicate metadata key");
        e.type = in_.scalar<uint32_t>();
        read_value(e);
        f_.meta.push_back(e);
    }

    void apply_alignment() {
        for (const MetaEntry &e : f_.meta) {
            if (f_.str(e.key_at, e.key_len) != "general.alignment") continue;
            expect(e.type == 4, "alignment must be uint32");
            expect(e.bits != 0 && e.bits <= (1u << 20) && (e.bits & (e.bits - 1)) == 0, "invalid alignment");
            f_.alignment = (uint32_t)e.bits;
        }
    }

    void read_tensor() {
        TensorEntry t{};
        std::tie(t.name_at, t.name_len) = kept_string();
        const std::string_view name = f_.str(t.name_at, t.name_len);
        expect(!name.empty() && name.find('\0') == std::string_view::npos, "invalid tensor name");
        expect(first_occurrence(t.name_at, t.name_len), "duplicate tensor name");
        t.rank = in_.scalar<uint32_t>();
        expect(t.rank >= 1 && t.rank <= kMaxRank, "invalid tensor rank");
        t.elements = 1;
        for (uint32_t d = 0; d < t.rank; ++d) {
            t.dims[d] = in_.scalar<uint64_t>();
            expect(t.dims[d] >= 1 && t.dims[d] <= INT32_MAX, "invalid tensor dimension");
            t.elements = product(t.elements, t.dims[d]);
        }
        t.type = in_.scalar<uint32_t>();
        const Geometry &g = geometry_of(t.type);
        expect(t.dims[0] % g.elements == 0, "continuous dimension is not block aligned");
        t.bytes = product(t.elements / g.elements, g.bytes);
        t.relative = in_.scalar<uint64_t>();
        expect(t.relative % f_.alignment == 0, "unaligned tensor offset");
        f_.tensors.push_back(t);
    }

    // Payloads start at the directory's end rounded up to the alignment; each must lie inside
    // the file (checked in directory order) and no two may overlap.
    void place_payloads() {
        f_.directory_end = in_.offset();
        const uint64_t a = f_.alignment;
        f_.data_offset = sum(f_.directory_end, a - 1) / a * a;
        expect(f_.data_offset <= f_.file_bytes, "missing aligned tensor data");
        for (TensorEntry &t : f_.tensors) {
            t.absolute = sum(f_.data_offset, t.relative);
            expect(t.absolute <= f_.file_bytes && t.bytes <= f_.file_bytes - t.absolute,
                   "tensor payload out of file bounds");
        }
        std::vector<uint32_t> order(f_.tensors.size());
        std::iota(order.begin(), order.end(), 0u);
        std::sort(order.begin(), order.end(), [&](uint32_t x, uint32_t y) {
            const TensorEntry &a = f_.tensors[x], &b = f_.tensors[y];
            return a.absolute != b.absolute ? a.absolute < b.absolute : a.bytes < b.bytes;
        });
        for (size_t i = 1; i < order.size(); ++i) {
            const TensorEntry &prev = f_.tensors[order[i - 1]], &cur = f_.tensors[order[i]];
            expect(cur.absolute >= prev.absolute + prev.bytes, "overlapping tensor payloads");
        }
    }

    tc_gguf_file &f_;
    DirectoryBytes in_;
    std::unordered_map<size_t, std::vector<std::pair<uint32_t, uint32_t>>> seen_;
};

// Split-set consistency, one shard at a time (gguf_directory.hpp:269-304 defines the rules
// and their order): every shard names its number (u16 split.no), the set size (u16
// split.count) and the total tensor count (i32 or u64 split.tensors.count); the numbers are
// distinct and below the set size, the counts and general.architecture agree, and the set's
// tensor names are unique and as many as announced. A lone file without split keys passes.
class SplitSet {
  public:
    explicit SplitSet(uint32_t size) : size_(size) {}

    // Returns false when the set is a lone file without split keys (nothing more to check).
    bool admit(const tc_gguf_file &f) {
        const MetaEntry *no = f.find_meta("split.no"), *total = f.find_meta("split.count");
        const MetaEntry *count = f.find_meta("split.tensors.count");
        if (size_ == 1 && !no && !total && !count) return false;
        expect(no && total && count && no->type == 2 && total->type == 2 && (count->type == 5 || count->type == 10),
               "invalid/missing split metadata");
        expect(total->bits == size_ && no->bits < size_, "missing split shard or invalid split number");
        expect(!(numbers_ >> no->bits & 1u), "duplicate split number");
        numbers_ |= 1ull << no->bits;
        expect(count->type != 5 || count->as_signed >= 0, "negative split tensor count");
        if (announced_ == 0) announced_ = count->bits;
        expect(announced_ != 0 && count->bits == announced_, "inconsistent split tensor count");
        const MetaEntry *arch = f.find_meta("general.architecture");
        expect(arch && arch->type == kString && arch->text_len != 0, "missing split architecture");
        const std::string_view a = f.str(arch->text_at, arch->text_len);
        if (arch_.empty()) arch_.assign(a);
        expect(arch_ == a, "inconsistent split architecture");
        for (const TensorEntry &t : f.tensors) {
            expect(names_.emplace(std::string(f.str(t.name_at, t.name_len))).second, "duplicate split tensor");
        }
        return true;
    }
    void finish() const { expect(names_.size() == announced_, "split tensor count mismatch"); }

  private:
    uint32_t size_;
    uint64_t numbers_ = 0;  // bit i: split.no i seen (the set holds at most 64 shards)
    uint64_t announced_ = 0;
    std::string arch_;
    std::unordered_set<std::string> names_;
};

void parse(tc_gguf_file &f) { DirectoryParser(f).run(); }

int fail(char **error, const std::string &msg) {
    if (error) *error = strdup(msg.c_str());
    return 1;
}

template <typename F>
int guarded(char **error, F &&body) {
    if (error) *error = nullptr;
    try {
        body();
        return 0;
    } catch (const std::exception &e) {
        return fail(error, e.what());
    } catch (...) {
        return fail(error, "unknown error");
    }
}

}  // namespace

extern "C" int tc_gguf_open(const char *path, tc_gguf_file **out, char **error) {
    if (out) *out = nullptr;
    return guarded(error, [&] {
        if (!path || !out) throw std::invalid_argument("null path or output handle");
        const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
        if (fd < 0) throw std::invalid_argument(std::string("gguf_open: ") + std::strerror(errno));
        auto *f = new tc_gguf_file();
        f->fd = fd;
        try {
            struct stat st;
            if (::fstat(fd, &st) != 0) throw std::invalid_argument(std::string("gguf_open: ") + std::strerror(errno));
            f->file_bytes = (uint64_t)st.st_size;
            parse(*f);
        } catch (...) {
            tc_gguf_close(f);
            throw;
        }
        *out = f;
    });
}

extern "C" void tc_gguf_close(tc_gguf_file *f) {
    if (!f) return;
    if (f->fd >= 0) ::close(f->fd);
    delete f;
}

extern "C" int tc_gguf_describe(const tc_gguf_file *f, tc_gguf_summary *out) {
    if (!f || !out) return 1;
    out->version = f->version;
    out->alignment = f->alignment;
    out->tensor_count = f->tensors.size();
    out->metadata_count = f->meta.size();
    out->file_bytes = f->file_bytes;
    out->data_offset = f->data_offset;
    return 0;
}

extern "C" int tc_gguf_tensor(const tc_gguf_file *f, uint64_t index, tc_gguf_tensor_info *out, char **error) {
    return guarded(error, [&] {
        if (!f || !out) throw std::invalid_argument("null handle or output");
        if (index >= f->tensors.size()) throw std::invalid_argument("tensor index out of range");
        const TensorEntry &t = f->tensors[index];
        std::memset(out, 0, sizeof *out);
        out->name = f->c_str(t.name_at);
        out->ggml_type = t.type;
        out->rank = t.rank;
        std::copy(t.dims, t.dims + t.rank, out->dims);
        out->elements = t.elements;
        out->bytes = t.bytes;
        out->file_offset = t.absolute;
        out->relative_offset = t.relative;
    });
}

extern "C" int tc_gguf_find_tensor(const tc_gguf_file *f, const char *name, uint64_t *index, char **error) {
    return guarded(error, [&] {
        if (!f || !name || !index) throw std::invalid_argument("null argument");
        const auto it = f->tensor_index.find(std::string_view(name));
        if (it == f->tensor_index.end()) throw std::invalid_argument(std::string("gguf_tensor_missing: ") + name);
        *index = it->second;
    });
}

extern "C" int tc_gguf_meta(const tc_gguf_file *f, const char *key, tc_gguf_meta_value *out, char **error) {
    return guarded(error, [&] {
        if (!f || !key || !out) throw std::invalid_argument("null argument");
        const MetaEntry *m = f->find_meta(key);
        if (!m) throw std::invalid_argument(std::string("gguf_metadata_missing: ") + key);
        std::memset(out, 0, sizeof *out);
        out->type = m->type;
        out->element_type = m->element_type;
        out->count = m->count;
        out->unsigned_value = m->bits;
        out->signed_value = m->as_signed;
        out->float_value = m->as_float;
        out->text = m->type == kString ? f->c_str(m->text_at) : "";
        out->text_bytes = m->type == kString ? m->text_len : 0;
    });
}

extern "C" int tc_gguf_validate_split(const tc_gguf_file *const *shards, uint32_t count, char **error) {
    return guarded(error, [&] {
        expect(shards && count && count <= 64, "empty/excessive split set");
        // Whole-set budgets first: the shards' tensors and retained directory bytes together
        // stay within one file's limits.
        uint64_t tensors = 0, retained = 0;
        for (uint32_t i = 0; i < count; ++i) {
            if (!shards[i]) throw std::invalid_argument("null shard");
            tensors = sum(tensors, shards[i]->tensors.size());
            retained = sum(retained, shards[i]->retained);
        }
        expect(tensors <= kMaxTensors && retained <= kMaxRetainedBytes, "aggregate split metadata limit");
        SplitSet set(count);
        for (uint32_t i = 0; i < count; ++i)
            if (!set.admit(*shards[i])) return;
        set.finish();
    });
}

// Tensor payload -> device memory: pread() into two pinned bounce buffers (4 MiB each,
// alternating, so a read overlaps the previous chunk's copy), hipMemcpyAsync on `stream`,
// synchronous on return.
extern "C" int tc_gguf_read_tensor(const tc_gguf_file *f, uint64_t index, void *device_dst, uint64_t dst_bytes,
                                   void *stream, char **error) {
    return guarded(error, [&] {
        if (!f || !device_dst) throw std::invalid_argument("null handle or destination");
        if (index >= f->tensors.size()) throw std::invalid_argument("tensor index out of range");
        const TensorEntry &t = f->tensors[index];
        if (dst_bytes < t.bytes) throw std::invalid_argument("destination buffer too short");
        const hipStream_t s = static_cast<hipStream_t>(stream);
        constexpr uint64_t kChunk = 4ull << 20;
        void *bounce[2] = {nullptr, nullptr};
        hipEvent_t done[2] = {nullptr, nullptr};
        auto release = [&] {
            for (int k = 0; k < 2; ++k) {
                if (done[k]) (void)hipEventSynchronize(done[k]), (void)hipEventDestroy(done[k]);
                if (bounce[k]) (void)hipHostFree(bounce[k]);
            }
        };
        try {
            for (int k = 0; k < 2; ++k) {
                if (hipHostMalloc(&bounce[k], kChunk, hipHostMallocDefault) != hipSuccess)
                    throw std::runtime_error("hipHostMalloc(bounce buffer) failed");
                if (hipEventCreateWithFlags(&done[k], hipEventDisableTiming) != hipSuccess)
                    throw std::runtime_error("hipEventCreate failed");
            }
            uint64_t off = 0;
            for (int k = 0; off < t.bytes; k ^= 1) {
                const uint64_t n = std::min(kChunk, t.bytes - off);
                if (hipEventSynchronize(done[k]) != hipSuccess) throw std::runtime_error("hipEventSynchronize failed");
                for (uint64_t got = 0; got < n;) {
                    const ssize_t r = ::pread(f->fd, static_cast<uint8_t *>(bounce[k]) + got, n - got,
                                              (off_t)(t.absolute + off + got));
                    if (r < 0 && errno == EINTR) continue;
                    if (r <= 0) throw std::runtime_error("gguf_read: tensor payload read failed or source changed");
                    got += (uint64_t)r;
                }
                if (hipMemcpyAsync(static_cast<uint8_t *>(device_dst) + off, bounce[k], n, hipMemcpyHostToDevice, s) !=
                        hipSuccess ||
                    hipEventRecord(done[k], s) != hipSuccess)
                    throw std::runtime_error("hipMemcpyAsync failed");
                off += n;
            }
            if (hipStreamSynchronize(s) != hipSuccess) throw std::runtime_error("hipStreamSynchronize failed");
        } catch (...) {
            release();
            throw;
        }
        release();
    });
}

// ---- weight pager: bounded device slots filled from the file ------------------------------
// Counterpart of the reference's GgufWeightPager fill / bind / retire
// (native/runtime/streaming/gguf_weight_pager.hpp:27-53) and of its slot safety tracker
// (slot_pool.hpp:11-45: Vacant -> Loading -> Ready -> InUse -> AwaitingFence), for models whose
// raw GGUF blocks do not all fit in device memory. A group (for example the projections of
// one transformer block) is filled into a slot as its raw tensor payloads, each at a 256-byte
// aligned offset; the kernels read them there directly. Fills run on a worker thread: pread()
// into two pinned bounce buffers and asynchronous copies on the pager's own copy stream, so
// that the reads and uploads of the next groups overlap the compute on the current one. The
// reader's stream waits for a fill's upload with a device-side event wait, and the next fill
// of a slot waits (on the copy stream) for the fence its last reader recorded.
namespace {

enum class SlotPhase { Vacant, Loading, Ready, Failed, InUse, AwaitingFence };

struct PagerSlot {
    uint8_t *base = nullptr;
    SlotPhase phase = SlotPhase::Vacant;
    uint64_t generation = 0;
    uint32_t group = 0;
    hipEvent_t uploaded = nullptr, fence = nullptr;
    bool fenced = false;  // `fence` holds the last reader's completion
    int status = 0;       // Failed: 1 error, 2 cancelled
    std::string error;
};

struct PagerJob {
    uint32_t slot;
    uint64_t generation;
    const volatile int *cancel;
};

constexpr uint64_t kPagerAlign = 256;
constexpr uint64_t kPagerChunk = 4ull << 20;

}  // namespace

struct tc_pager {
    const tc_gguf_file *file = nullptr;
    int device = 0;
    hipStream_t copy = nullptr;
    std::vector<std::vector<uint32_t>> groups;       // tensor indices per group
    std::vector<std::vector<uint64_t>> offsets;      // their offsets in a slot
    std::vector<uint64_t> group_bytes;
    uint64_t slot_bytes = 0;
    std::vector<PagerSlot> slots;
    void *bounce[2] = {nullptr, nullptr};
    hipEvent_t bounce_done[2] = {nullptr, nullptr};
    std::mutex mu;
    std::condition_variable cv;
    std::deque<PagerJob> queue;
    bool stop = false;
    std::thread worker;
    tc_pager_metrics metrics{};

    void run();
    void fill_slot(const PagerJob &job);
};

namespace {

void hip_ok(hipError_t e, const char *what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

struct PagerCancelled : std::runtime_error {
    using std::runtime_error::runtime_error;
};

}  // namespace

void tc_pager::fill_slot(const PagerJob &job) {
    PagerSlot &s = slots[job.slot];
    const uint32_t g = s.group;
    const auto t0 = std::chrono::steady_clock::now();
    // The last reader of this slot must be done before its bytes are overwritten.
    if (s.fenced) hip_ok(hipStreamWaitEvent(copy, s.fence, 0), "hipStreamWaitEvent(reader fence)");
    int k = 0;
    uint64_t read = 0;
    for (size_t i = 0; i < groups[g].size(); ++i) {
        const TensorEntry &t = file->tensors[groups[g][i]];
        for (uint64_t off = 0; off < t.bytes; k ^= 1) {
            if (job.cancel && *job.cancel) throw PagerCancelled("gguf_pager: fill cancelled");
            const uint64_t n = std::min(kPagerChunk, t.bytes - off);
            hip_ok(hipEventSynchronize(bounce_done[k]), "hipEventSynchronize(bounce buffer)");
            for (uint64_t got = 0; got < n;) {
                const ssize_t r = ::pread(file->fd, static_cast<uint8_t *>(bounce[k]) + got, n - got,
                                          (off_t)(t.absolute + off + got));
                if (r < 0 && errno == EINTR) continue;
                if (r <= 0) throw std::runtime_error("gguf_pager: payload read failed or source changed");
                got += (uint64_t)r;
            }
            hip_ok(hipMemcpyAsync(s.base + offsets[g][i] + off, bounce[k], n, hipMemcpyHostToDevice, copy),
                   "hipMemcpyAsync(slot upload)");
            hip_ok(hipEventRecord(bounce_done[k], copy), "hipEventRecord(bounce buffer)");
            off += n;
            read += n;
        }
    }
    hip_ok(hipEventRecord(s.uploaded, copy), "hipEventRecord(upload)");
    std::lock_guard<std::mutex> lock(mu);
    metrics.fills += 1;
    metrics.bytes_read += read;
    metrics.read_seconds += std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
}

void tc_pager::run() {
    (void)hipSetDevice(device);
    for (;;) {
        PagerJob job;
        {
            std::unique_lock<std::mutex> lock(mu);
            cv.wait(lock, [&] { return stop || !queue.empty(); });
            if (queue.empty()) return;  // stop with nothing left
            job = queue.front();
            queue.pop_front();
        }
        int status = 0;
        std::string error;
        try {
            fill_slot(job);
        } catch (const PagerCancelled &e) {
            status = 2;
            error = e.what();
        } catch (const std::exception &e) {
            status = 1;
            error = e.what();
        }
        std::lock_guard<std::mutex> lock(mu);
        PagerSlot &s = slots[job.slot];
        if (s.generation == job.generation) {
            s.phase = status ? SlotPhase::Failed : SlotPhase::Ready;
            s.status = status;
            s.error = error;
        }
        cv.notify_all();
    }
}

namespace {

int pager_status(char **error, int status, const std::string &msg) {
    if (error) *error = strdup(msg.c_str());
    return status;
}

PagerSlot &ticket_slot(tc_pager *p, const tc_pager_ticket *t) {
    if (!p || !t) throw std::invalid_argument("null pager or ticket");
    if (t->slot >= p->slots.size()) throw std::invalid_argument("gguf_pager: slot out of range");
    PagerSlot &s = p->slots[t->slot];
    if (s.generation != t->generation || s.group != t->group)
        throw std::invalid_argument("gguf_pager: stale slot ticket");
    return s;
}

}  // namespace

extern "C" int tc_pager_create(const tc_gguf_file *file, uint32_t group_count, const uint32_t *group_begin,
                               const uint64_t *tensor_indices, uint32_t slot_count, void *const *slot_buffers,
                               uint64_t slot_bytes, tc_pager **out, char **error) {
    if (out) *out = nullptr;
    return guarded(error, [&] {
        if (!file || !out || !group_begin || !slot_buffers) throw std::invalid_argument("null argument");
        if (group_count == 0 || slot_count == 0) throw std::invalid_argument("gguf_pager: no groups or no slots");
        auto p = std::make_unique<tc_pager>();
        p->file = file;
        p->slot_bytes = slot_bytes;
        hip_ok(hipGetDevice(&p->device), "hipGetDevice");
        for (uint32_t g = 0; g < group_count; ++g) {
            if (group_begin[g + 1] < group_begin[g]) throw std::invalid_argument("gguf_pager: invalid group table");
            std::vector<uint32_t> idx;
            std::vector<uint64_t> off;
            uint64_t at = 0;
            for (uint32_t i = group_begin[g]; i < group_begin[g + 1]; ++i) {
                if (!tensor_indices || tensor_indices[i] >= file->tensors.size())
                    throw std::invalid_argument("gguf_pager: tensor index out of range");
                idx.push_back((uint32_t)tensor_indices[i]);
                off.push_back(at);
                at = sum(at, file->tensors[tensor_indices[i]].bytes);
                at = (at + kPagerAlign - 1) / kPagerAlign * kPagerAlign;
            }
            if (at > slot_bytes) throw std::invalid_argument("gguf_pager: group larger than a slot");
            p->groups.push_back(std::move(idx));
            p->offsets.push_back(std::move(off));
            p->group_bytes.push_back(at);
        }
        p->slots.resize(slot_count);
        struct Cleanup {
            tc_pager *p;
            bool armed = true;
            ~Cleanup() {
                if (!armed) return;
                for (auto &s : p->slots) {
                    if (s.uploaded) (void)hipEventDestroy(s.uploaded);
                    if (s.fence) (void)hipEventDestroy(s.fence);
                }
                for (int k = 0; k < 2; ++k) {
                    if (p->bounce_done[k]) (void)hipEventDestroy(p->bounce_done[k]);
                    if (p->bounce[k]) (void)hipHostFree(p->bounce[k]);
                }
                if (p->copy) (void)hipStreamDestroy(p->copy);
            }
        } cleanup{p.get()};
        for (uint32_t i = 0; i < slot_count; ++i) {
            if (!slot_buffers[i] || (reinterpret_cast<uintptr_t>(slot_buffers[i]) & (kPagerAlign - 1)))
                throw std::invalid_argument("gguf_pager: slot buffers must be 256-byte aligned device memory");
            p->slots[i].base = static_cast<uint8_t *>(slot_buffers[i]);
            hip_ok(hipEventCreateWithFlags(&p->slots[i].uploaded, hipEventDisableTiming), "hipEventCreate");
            hip_ok(hipEventCreateWithFlags(&p->slots[i].fence, hipEventDisableTiming), "hipEventCreate");
        }
        for (int k = 0; k < 2; ++k) {
            hip_ok(hipHostMalloc(&p->bounce[k], kPagerChunk, hipHostMallocDefault), "hipHostMalloc(bounce buffer)");
            hip_ok(hipEventCreateWithFlags(&p->bounce_done[k], hipEventDisableTiming), "hipEventCreate");
        }
        hip_ok(hipStreamCreateWithFlags(&p->copy, hipStreamNonBlocking), "hipStreamCreate(copy)");
        p->worker = std::thread([pp = p.get()] { pp->run(); });
        cleanup.armed = false;
        *out = p.release();
    });
}

extern "C" int tc_pager_group_layout(const tc_pager *p, uint32_t group, uint64_t *offsets, uint32_t capacity,
                                     uint32_t *count, uint64_t *bytes, char **error) {
    return guarded(error, [&] {
        if (!p || !count) throw std::invalid_argument("null pager or output");
        if (group >= p->groups.size()) throw std::invalid_argument("gguf_pager: group out of range");
        *count = (uint32_t)p->groups[group].size();
        if (bytes) *bytes = p->group_bytes[group];
        if (offsets) {
            if (capacity < *count) throw std::invalid_argument("gguf_pager: offset array too short");
            std::copy(p->offsets[group].begin(), p->offsets[group].end(), offsets);
        }
    });
}

extern "C" int tc_pager_fill(tc_pager *p, uint32_t group, uint32_t slot, const volatile int *cancel,
                             tc_pager_ticket *ticket, char **error) {
    return guarded(error, [&] {
        if (!p || !ticket) throw std::invalid_argument("null pager or ticket");
        if (group >= p->groups.size()) throw std::invalid_argument("gguf_pager: group out of range");
        if (slot >= p->slots.size()) throw std::invalid_argument("gguf_pager: slot out of range");
        std::lock_guard<std::mutex> lock(p->mu);
        PagerSlot &s = p->slots[slot];
        if (s.phase != SlotPhase::Vacant && s.phase != SlotPhase::AwaitingFence)
            throw std::invalid_argument("gguf_pager: slot is not vacant");
        s.phase = SlotPhase::Loading;
        s.generation += 1;
        s.group = group;
        s.status = 0;
        s.error.clear();
        p->queue.push_back(PagerJob{slot, s.generation, cancel});
        *ticket = tc_pager_ticket{group, slot, s.generation};
        p->cv.notify_all();
    });
}

extern "C" int tc_pager_acquire(tc_pager *p, const tc_pager_ticket *ticket, void *stream, char **error) {
    if (error) *error = nullptr;
    if (!p || !ticket) return pager_status(error, 1, "null pager or ticket");
    try {
        std::unique_lock<std::mutex> lock(p->mu);
        PagerSlot &s = ticket_slot(p, ticket);
        const auto t0 = std::chrono::steady_clock::now();
        p->cv.wait(lock, [&] { return s.phase != SlotPhase::Loading || s.generation != ticket->generation; });
        p->metrics.wait_seconds += std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        if (s.generation != ticket->generation) throw std::invalid_argument("gguf_pager: stale slot ticket");
        if (s.phase == SlotPhase::Failed) {
            const int status = s.status;
            const std::string msg = s.error;
            s.phase = SlotPhase::Vacant;  // the slot's bytes are undefined; it may be filled again
            return pager_status(error, status, msg);
        }
        if (s.phase != SlotPhase::Ready) throw std::invalid_argument("gguf_pager: slot is not ready");
        s.phase = SlotPhase::InUse;
        hipEvent_t up = s.uploaded;
        lock.unlock();
        if (stream) hip_ok(hipStreamWaitEvent(static_cast<hipStream_t>(stream), up, 0), "hipStreamWaitEvent(upload)");
        else hip_ok(hipEventSynchronize(up), "hipEventSynchronize(upload)");
        return 0;
    } catch (const std::exception &e) {
        return pager_status(error, 1, e.what());
    }
}

extern "C" int tc_pager_release(tc_pager *p, const tc_pager_ticket *ticket, void *stream, char **error) {
    return guarded(error, [&] {
        if (!p || !ticket) throw std::invalid_argument("null pager or ticket");
        std::lock_guard<std::mutex> lock(p->mu);
        PagerSlot &s = ticket_slot(p, ticket);
        if (s.phase != SlotPhase::InUse) throw std::invalid_argument("gguf_pager: slot is not in use");
        hip_ok(hipEventRecord(s.fence, static_cast<hipStream_t>(stream)), "hipEventRecord(reader fence)");
        s.fenced = true;
        s.phase = SlotPhase::AwaitingFence;
    });
}

extern "C" int tc_pager_get_metrics(tc_pager *p, tc_pager_metrics *out) {
    if (!p || !out) return 1;
    std::lock_guard<std::mutex> lock(p->mu);
    *out = p->metrics;
    return 0;
}

extern "C" void tc_pager_free(tc_pager *p) {
    if (!p) return;
    {
        std::lock_guard<std::mutex> lock(p->mu);
        p->stop = true;
        p->cv.notify_all();
    }
    if (p->worker.joinable()) p->worker.join();  // finishes the queued fills
    (void)hipStreamSynchronize(p->copy);
    for (auto &s : p->slots) {
        if (s.uploaded) (void)hipEventDestroy(s.uploaded);
        if (s.fence) (void)hipEventDestroy(s.fence);
    }
    for (int k = 0; k < 2; ++k) {
        if (p->bounce_done[k]) (void)hipEventDestroy(p->bounce_done[k]);
        if (p->bounce[k]) (void)hipHostFree(p->bounce[k]);
    }
    (void)hipStreamDestroy(p->copy);
    delete p;
}
