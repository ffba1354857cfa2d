// GGUF container reader: directory parse and raw tensor upload to device memory.
//
// Counterpart of the reference's directory reader tc::gguf::read_directory and
// validate_split_set (native/core/gguf_directory.hpp:199-304; type table :19-26, limits
// :45-50). The same file format checks and error strings ("gguf_invalid: <reason>"), the
// same limits, and the same derived geometry (data offset aligned up to general.alignment,
// payload bytes from the block table, bounds and overlap checks). Host code only: tensor
// payloads are read with pread() into pinned bounce buffers and copied to device with
// hipMemcpyAsync, so a Q4_K / Q6_K weight arrives in HBM as the raw blocks the kernels
// consume (no host-side decode).
#include "../../include/tc_qlinear.h"

#include <hip/hip_runtime.h>

#include <errno.h>
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <unordered_set>
#include <utility>
#include <vector>

namespace {

struct BlockType {
    uint32_t id, elements, bytes;
    const char *name;
};
// GGML tensor type ids the reader accepts (gguf_directory.hpp:21-26).
constexpr BlockType kTypes[] = {{0, 1, 4, "F32"},    {1, 1, 2, "F16"},      {2, 32, 18, "Q4_0"},
                                {3, 32, 20, "Q4_1"}, {6, 32, 22, "Q5_0"},   {7, 32, 24, "Q5_1"},
                                {8, 32, 34, "Q8_0"}, {12, 256, 144, "Q4_K"}, {13, 256, 176, "Q5_K"},
                                {14, 256, 210, "Q6_K"}, {30, 1, 2, "BF16"}};

const BlockType &block_type(uint32_t id) {
    for (const BlockType &t : kTypes)
        if (t.id == id) return t;
    throw std::invalid_argument("gguf_type_unsupported: " + std::to_string(id));
}

void check(bool ok, const char *reason) {
    if (!ok) throw std::invalid_argument(std::string("gguf_invalid: ") + reason);
}
uint64_t add(uint64_t a, uint64_t b) {
    check(b <= UINT64_MAX - a, "integer addition overflow");
    return a + b;
}
uint64_t mul(uint64_t a, uint64_t b) {
    check(!a || b <= UINT64_MAX / a, "integer multiplication overflow");
    return a * b;
}

// Parser limits (gguf_directory.hpp:45-50).
struct Limits {
    uint64_t tensors = 65536, metadata_entries = 65536;
    uint64_t directory_bytes = 64ull << 20, retained_bytes = 32ull << 20;
    uint64_t string_bytes = 1ull << 20, array_elements = 1ull << 20;
    uint32_t max_rank = 4, max_array_depth = 4;
};

struct Meta {
    std::string key, text;
    uint32_t type = 0, element_type = 0;
    uint64_t count = 0, u = 0;
    int64_t i = 0;
    double f = 0;
};

struct Tensor {
    std::string name;
    uint32_t type = 0;
    std::vector<uint64_t> dims;  // GGML order: dims[0] contiguous
    uint64_t relative_offset = 0, file_offset = 0, bytes = 0, elements = 0;
};

// Sequential little-endian reader over a file descriptor with a 64 KiB read-ahead window;
// every read is bounds-checked against the file size and the directory byte limit.
class Cursor {
  public:
    Cursor(int fd, uint64_t size, const Limits &lim) : fd_(fd), size_(size), lim_(lim), window_(1 << 16) {}
    uint64_t pos() const { return pos_; }
    uint64_t retained() const { return retained_; }
    void charge(uint64_t bytes) {
        retained_ = add(retained_, bytes);
        check(retained_ <= lim_.retained_bytes, "retained metadata limit");
    }
    void skip(uint64_t bytes) {
        check(pos_ <= size_ && bytes <= size_ - pos_, "truncated directory");
        check(pos_ <= lim_.directory_bytes && bytes <= lim_.directory_bytes - pos_, "directory byte limit");
        pos_ += bytes;
    }
    void read(void *dst, uint64_t bytes) {
        const uint64_t start = pos_;
        skip(bytes);
        uint8_t *out = static_cast<uint8_t *>(dst);
        for (uint64_t done = 0; done < bytes;) {
            const uint64_t at = start + done;
            if (at >= wbeg_ && at < wbeg_ + wlen_) {
                const uint64_t n = std::min<uint64_t>(bytes - done, wbeg_ + wlen_ - at);
                std::memcpy(out + done, window_.data() + (at - wbeg_), n);
                done += n;
                continue;
            }
            const uint64_t want = std::min<uint64_t>(window_.size(), std::min(size_, lim_.directory_bytes) - at);
            const ssize_t n = ::pread(fd_, window_.data(), want, (off_t)at);
            if (n < 0 && errno == EINTR) continue;
            check(n > 0, "directory read failed or source changed");
            wbeg_ = at;
            wlen_ = (uint64_t)n;
        }
    }
    uint64_t uint(uint32_t width) {
        uint8_t b[8] = {};
        read(b, width);
        uint64_t v = 0;
        for (uint32_t k = 0; k < width; ++k) v |= (uint64_t)b[k] << (8 * k);
        return v;
    }
    std::string str(bool keep) {
        const uint64_t n = uint(8);
        check(n <= lim_.string_bytes, "string byte limit");
        if (!keep) {
            skip(n);
            return {};
        }
        charge(add(n, 1));
        std::string s((size_t)n, '\0');
        read(s.data(), n);
        return s;
    }
    // One metadata value of `type` (GGUF value types 0..12), stored into `m` when given;
    // array payloads are skipped (strings and nested arrays element by element).
    void value(uint32_t type, Meta *m, uint32_t depth = 0) {
        if (type == 8) {
            std::string s = str(m != nullptr);
            if (m) m->text = std::move(s);
            return;
        }
        if (type == 9) {
            check(depth < lim_.max_array_depth, "nested array depth limit");
            const uint32_t et = (uint32_t)uint(4);
            const uint64_t count = uint(8);
            check(count <= lim_.array_elements, "array element limit");
            check(et <= 12, "invalid array element type");
            if (m) {
                m->element_type = et;
                m->count = count;
            }
            if (et == 7 || et == 8 || et == 9) {
                for (uint64_t k = 0; k < count; ++k) value(et, nullptr, depth + 1);
            } else {
                skip(mul(count, width_of(et)));
            }
            return;
        }
        const uint32_t w = width_of(type);
        const uint64_t bits = uint(w);
        if (type == 7) check(bits <= 1, "invalid boolean");
        if (!m) return;
        m->u = bits;
        if (type == 1 || type == 3 || type == 5 || type == 11) {
            const uint64_t sign = 1ull << (8 * w - 1);
            m->i = (int64_t)((w < 8 && (bits & sign)) ? (bits | (~0ull << (8 * w))) : bits);
        }
        if (type == 6) {
            float f;
            const uint32_t b32 = (uint32_t)bits;
            std::memcpy(&f, &b32, 4);
            m->f = f;
        }
        if (type == 12) std::memcpy(&m->f, &bits, 8);
    }

  private:
    static uint32_t width_of(uint32_t type) {
        switch (type) {
        case 0: case 1: case 7: return 1;
        case 2: case 3: return 2;
        case 4: case 5: case 6: return 4;
        case 10: case 11: case 12: return 8;
        default: throw std::invalid_argument("gguf_invalid: invalid metadata scalar type");
        }
    }
    int fd_;
    uint64_t size_, pos_ = 0, retained_ = 0;
    const Limits &lim_;
    std::vector<uint8_t> window_;
    uint64_t wbeg_ = 0, wlen_ = 0;
};

}  // namespace

struct tc_gguf_file {
    int fd = -1;
    uint64_t file_bytes = 0;
    uint32_t version = 0, alignment = 32;
    uint64_t directory_end = 0, data_offset = 0;
    std::vector<Meta> meta;
    std::vector<Tensor> tensors;
};

namespace {

void parse(tc_gguf_file &f) {
    const Limits lim;
    Cursor c(f.fd, f.file_bytes, lim);
    check(c.uint(4) == 0x46554747u, "invalid GGUF magic/endian");
    f.version = (uint32_t)c.uint(4);
    check(f.version == 2 || f.version == 3, "unsupported GGUF version");
    const uint64_t n_tensors = c.uint(8), n_meta = c.uint(8);
    check(n_tensors && n_tensors <= lim.tensors && n_tensors <= f.file_bytes / 24, "tensor count limit");
    check(n_meta <= lim.metadata_entries && n_meta <= f.file_bytes / 12, "metadata count limit");
    c.charge(mul(n_tensors, sizeof(Tensor) + 256));
    c.charge(mul(n_meta, sizeof(Meta) + 128));
    std::unordered_set<std::string> seen;
    for (uint64_t k = 0; k < n_meta; ++k) {
        Meta m;
        m.key = c.str(true);
        check(!m.key.empty() && m.key.find('\0') == std::string::npos, "invalid metadata key");
        c.charge(m.key.size() + 1);
        check(seen.insert(m.key).second, "duplicate metadata key");
        m.type = (uint32_t)c.uint(4);
        c.value(m.type, &m);
        f.meta.push_back(std::move(m));
    }
    for (const Meta &m : f.meta) {
        if (m.key != "general.alignment") continue;
        check(m.type == 4, "alignment must be uint32");
        check(m.u && m.u <= (1u << 20) && !(m.u & (m.u - 1)), "invalid alignment");
        f.alignment = (uint32_t)m.u;
    }
    seen.clear();
    for (uint64_t k = 0; k < n_tensors; ++k) {
        Tensor t;
        t.name = c.str(true);
        check(!t.name.empty() && t.name.find('\0') == std::string::npos, "invalid tensor name");
        c.charge(t.name.size() + 1);
        check(seen.insert(t.name).second, "duplicate tensor name");
        const uint32_t rank = (uint32_t)c.uint(4);
        check(rank && rank <= lim.max_rank, "invalid tensor rank");
        t.elements = 1;
        for (uint32_t r = 0; r < rank; ++r) {
            const uint64_t d = c.uint(8);
            check(d && d <= INT32_MAX, "invalid tensor dimension");
            t.elements = mul(t.elements, d);
            t.dims.push_back(d);
        }
        t.type = (uint32_t)c.uint(4);
        const BlockType &bt = block_type(t.type);
        check(t.dims[0] % bt.elements == 0, "continuous dimension is not block aligned");
        t.bytes = mul(t.elements / bt.elements, bt.bytes);
        t.relative_offset = c.uint(8);
        check(t.relative_offset % f.alignment == 0, "unaligned tensor offset");
        f.tensors.push_back(std::move(t));
    }
    f.directory_end = c.pos();
    const uint64_t mask = f.alignment - 1;
    f.data_offset = add(f.directory_end, mask) & ~mask;
    check(f.data_offset <= f.file_bytes, "missing aligned tensor data");
    std::vector<std::pair<uint64_t, uint64_t>> spans;
    for (Tensor &t : f.tensors) {
        t.file_offset = add(f.data_offset, t.relative_offset);
        check(t.file_offset <= f.file_bytes && t.bytes <= f.file_bytes - t.file_offset,
              "tensor payload out of file bounds");
        spans.emplace_back(t.file_offset, add(t.file_offset, t.bytes));
    }
    std::sort(spans.begin(), spans.end());
    for (size_t k = 1; k < spans.size(); ++k) check(spans[k].first >= spans[k - 1].second, "overlapping tensor payloads");
}

const Meta *find_meta(const tc_gguf_file &f, const char *key) {
    for (const Meta &m : f.meta)
        if (m.key == key) return &m;
    return nullptr;
}

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
        const Tensor &t = f->tensors[index];
        std::memset(out, 0, sizeof *out);
        out->name = t.name.c_str();
        out->ggml_type = t.type;
        out->rank = (uint32_t)t.dims.size();
        for (size_t r = 0; r < t.dims.size(); ++r) out->dims[r] = t.dims[r];
        out->elements = t.elements;
        out->bytes = t.bytes;
        out->file_offset = t.file_offset;
        out->relative_offset = t.relative_offset;
    });
}

extern "C" int tc_gguf_find_tensor(const tc_gguf_file *f, const char *name, uint64_t *index, char **error) {
    return guarded(error, [&] {
        if (!f || !name || !index) throw std::invalid_argument("null argument");
        for (size_t k = 0; k < f->tensors.size(); ++k)
            if (f->tensors[k].name == name) {
                *index = k;
                return;
            }
        throw std::invalid_argument(std::string("gguf_tensor_missing: ") + name);
    });
}

extern "C" int tc_gguf_meta(const tc_gguf_file *f, const char *key, tc_gguf_meta_value *out, char **error) {
    return guarded(error, [&] {
        if (!f || !key || !out) throw std::invalid_argument("null argument");
        const Meta *m = find_meta(*f, key);
        if (!m) throw std::invalid_argument(std::string("gguf_metadata_missing: ") + key);
        std::memset(out, 0, sizeof *out);
        out->type = m->type;
        out->element_type = m->element_type;
        out->count = m->count;
        out->unsigned_value = m->u;
        out->signed_value = m->i;
        out->float_value = m->f;
        out->text = m->text.c_str();
        out->text_bytes = m->text.size();
    });
}

// Split sets (gguf_directory.hpp:269-304): every shard carries split.no (u16), split.count
// (u16) and split.tensors.count (i32 or u64), numbers are distinct and cover the set, the
// architecture agrees, tensor names are unique across shards and their count matches.
extern "C" int tc_gguf_validate_split(const tc_gguf_file *const *shards, uint32_t count, char **error) {
    return guarded(error, [&] {
        const Limits lim;
        check(shards && count && count <= 64, "empty/excessive split set");
        uint64_t tensors = 0;
        for (uint32_t s = 0; s < count; ++s) {
            if (!shards[s]) throw std::invalid_argument("null shard");
            tensors = add(tensors, shards[s]->tensors.size());
        }
        check(tensors <= lim.tensors, "aggregate split metadata limit");
        std::unordered_set<uint64_t> numbers;
        std::unordered_set<std::string> names;
        std::string arch;
        uint64_t expect = 0;
        for (uint32_t s = 0; s < count; ++s) {
            const tc_gguf_file &f = *shards[s];
            const Meta *no = find_meta(f, "split.no"), *total = find_meta(f, "split.count");
            const Meta *tc = find_meta(f, "split.tensors.count");
            if (count == 1 && !no && !total && !tc) return;
            check(no && total && tc && no->type == 2 && total->type == 2 && (tc->type == 5 || tc->type == 10),
                  "invalid/missing split metadata");
            check(total->u == count && no->u < count, "missing split shard or invalid split number");
            check(numbers.insert(no->u).second, "duplicate split number");
            check(tc->type != 5 || tc->i >= 0, "negative split tensor count");
            if (!expect) expect = tc->u;
            check(expect && tc->u == expect, "inconsistent split tensor count");
            const Meta *a = find_meta(f, "general.architecture");
            check(a && a->type == 8 && !a->text.empty(), "missing split architecture");
            if (arch.empty()) arch = a->text;
            check(arch == a->text, "inconsistent split architecture");
            for (const Tensor &t : f.tensors) check(names.insert(t.name).second, "duplicate split tensor");
        }
        check(names.size() == expect, "split tensor count mismatch");
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
        const Tensor &t = f->tensors[index];
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
                                              (off_t)(t.file_offset + off + got));
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
