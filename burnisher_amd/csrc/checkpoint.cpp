// Checkpoint input for the dit-step: safetensors shards memory-mapped read-only, their JSON
// headers parsed, and the DiT's tensors converted to bf16 and uploaded into one device arena.
//
// Reference behaviour followed (src/core/safetensors.cpp, src/models/weights.cpp):
//   - a shard is `u64 header_len | JSON header | data`; the header maps each tensor name to
//     {dtype, shape, data_offsets: [begin, end)} relative to the end of the header, plus an
//     optional "__metadata__" entry that is skipped (safetensors.cpp:225-247);
//   - dtypes F32, BF16, F16 and F8_E4M3 are recognised, anything else is refused at open
//     (safetensors.cpp:186-195); a byte range that disagrees with its shape, or runs past the end
//     of the file, is refused at open (safetensors.cpp:236-245);
//   - a component is the sorted list of `*.safetensors` files in `<dir>/<name>/`
//     (weights.cpp:26-49); a name is looked up shard by shard, and a miss reports the near
//     misses of the first shard (weights.cpp:56-65, safetensors.cpp:256-280);
//   - conversion to the compute dtype is per element through float: fp32 -> bf16 with
//     round-to-nearest-even (tensor.cpp:142-150); F16 and F8_E4M3 have no scalar accessor in
//     the reference (tensor.cpp:68-82) and are refused the same way here;
//   - device weights are converted on the host into page-locked staging and copied once
//     (weights.cpp:198-217). Here every DiT tensor lands in one arena allocated once, and the
//     conversion of one chunk overlaps the copy of the previous one.
// The JSON reader is this file's own: recursive descent over the grammar of RFC 8259, enough
// for a safetensors header.
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cctype>
#include <cmath>
#include <cstring>
#include <dirent.h>
#include <map>
#include <memory>
#include <string>
#include <thread>
#include <vector>

#include "../../include/burnisher_hip.h"
#include "common.h"

namespace bh {
namespace {

// ---- JSON ---------------------------------------------------------------------------------

struct Json {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    bool b = false;
    double num = 0.0;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;   // in document order

    const Json* find(const std::string& key) const {
        for (const auto& kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

class JsonReader {
  public:
    explicit JsonReader(const char* p, size_t n) : p_(p), n_(n) {}

    Json document() {
        Json v = value(0);
        skip_ws();
        if (i_ != n_) fail("content after the top-level value");
        return v;
    }

  private:
    const char* p_;
    size_t n_;
    size_t i_ = 0;

    [[noreturn]] void fail(const std::string& what) const {
        throw Error("json: " + what + " at byte " + std::to_string(i_));
    }
    void skip_ws() {
        while (i_ < n_ && (p_[i_] == ' ' || p_[i_] == '\t' || p_[i_] == '\n' || p_[i_] == '\r')) ++i_;
    }
    char next_char() {
        skip_ws();
        if (i_ >= n_) fail("unexpected end of text");
        return p_[i_];
    }
    void literal(const char* word) {
        const size_t len = std::strlen(word);
        if (n_ - i_ < len || std::memcmp(p_ + i_, word, len) != 0) fail("unknown literal");
        i_ += len;
    }

    Json value(int depth) {
        if (depth > 64) fail("nesting deeper than 64");
        Json v;
        switch (next_char()) {
            case '{': {
                ++i_;
                v.kind = Json::OBJ;
                if (next_char() == '}') { ++i_; return v; }
                for (;;) {
                    if (next_char() != '"') fail("expected a string key");
                    std::string key = string();
                    if (next_char() != ':') fail("expected ':'");
                    ++i_;
                    v.obj.emplace_back(std::move(key), value(depth + 1));
                    const char c = next_char();
                    ++i_;
                    if (c == '}') return v;
                    if (c != ',') fail("expected ',' or '}'");
                }
            }
            case '[': {
                ++i_;
                v.kind = Json::ARR;
                if (next_char() == ']') { ++i_; return v; }
                for (;;) {
                    v.arr.push_back(value(depth + 1));
                    const char c = next_char();
                    ++i_;
                    if (c == ']') return v;
                    if (c != ',') fail("expected ',' or ']'");
                }
            }
            case '"':
                v.kind = Json::STR;
                v.str = string();
                return v;
            case 't': literal("true"); v.kind = Json::BOOL; v.b = true; return v;
            case 'f': literal("false"); v.kind = Json::BOOL; return v;
            case 'n': literal("null"); return v;
            default:
                v.kind = Json::NUM;
                v.num = number();
                return v;
        }
    }

    double number() {
        const size_t start = i_;
        if (i_ < n_ && p_[i_] == '-') ++i_;
        const auto digits = [&]() {
            const size_t s = i_;
            while (i_ < n_ && std::isdigit(static_cast<unsigned char>(p_[i_]))) ++i_;
            return i_ > s;
        };
        if (!digits()) fail("expected a value");
        if (i_ < n_ && p_[i_] == '.') {
            ++i_;
            if (!digits()) fail("expected digits after '.'");
        }
        if (i_ < n_ && (p_[i_] == 'e' || p_[i_] == 'E')) {
            ++i_;
            if (i_ < n_ && (p_[i_] == '+' || p_[i_] == '-')) ++i_;
            if (!digits()) fail("expected an exponent");
        }
        return std::strtod(std::string(p_ + start, i_ - start).c_str(), nullptr);
    }

    static void put_utf8(std::string& out, uint32_t cp) {
        if (cp < 0x80) {
            out += static_cast<char>(cp);
        } else if (cp < 0x800) {
            out += static_cast<char>(0xC0 | (cp >> 6));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            out += static_cast<char>(0xE0 | (cp >> 12));
            out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        } else {
            out += static_cast<char>(0xF0 | (cp >> 18));
            out += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
            out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        }
    }

    uint32_t hex4() {
        if (n_ - i_ < 4) fail("truncated \\u escape");
        uint32_t cp = 0;
        for (int k = 0; k < 4; ++k) {
            const char c = p_[i_++];
            cp <<= 4;
            if (c >= '0' && c <= '9') cp |= c - '0';
            else if (c >= 'a' && c <= 'f') cp |= c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') cp |= c - 'A' + 10;
            else fail("bad hex digit in \\u escape");
        }
        return cp;
    }

    std::string string() {
        ++i_;   // the opening quote
        std::string out;
        while (i_ < n_) {
            const char c = p_[i_++];
            if (c == '"') return out;
            if (static_cast<unsigned char>(c) < 0x20) fail("control character in a string");
            if (c != '\\') {
                out += c;
                continue;
            }
            if (i_ >= n_) fail("unterminated escape");
            const char e = p_[i_++];
            switch (e) {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    uint32_t cp = hex4();
                    if (cp >= 0xD800 && cp < 0xDC00 && n_ - i_ >= 6 && p_[i_] == '\\' &&
                        p_[i_ + 1] == 'u') {   // a surrogate pair
                        i_ += 2;
                        const uint32_t lo = hex4();
                        if (lo < 0xDC00 || lo >= 0xE000) fail("unpaired surrogate");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    put_utf8(out, cp);
                    break;
                }
                default: fail("unknown escape");
            }
        }
        fail("unterminated string");
    }
};

// ---- one shard ----------------------------------------------------------------------------

// Element types of a safetensors file that this library names (the bh_st_dtype codes).
enum StDtype { ST_F32 = 0, ST_BF16 = 1, ST_F16 = 2, ST_F8_E4M3 = 3 };

const char* st_dtype_name(int t) {
    switch (t) {
        case ST_F32: return "F32";
        case ST_BF16: return "BF16";
        case ST_F16: return "F16";
        case ST_F8_E4M3: return "F8_E4M3";
    }
    return "?";
}
int st_dtype_bytes(int t) { return t == ST_F32 ? 4 : t == ST_F8_E4M3 ? 1 : 2; }

int st_dtype_parse(const std::string& s, const std::string& tensor) {
    if (s == "F32") return ST_F32;
    if (s == "BF16") return ST_BF16;
    if (s == "F16") return ST_F16;
    if (s == "F8_E4M3") return ST_F8_E4M3;
    throw Error("safetensors: " + tensor + " has dtype '" + s +
                "', which this library does not read (F32, BF16, F16, F8_E4M3). A checkpoint "
                "converted silently would no longer be the one the oracle was pinned on.");
}

struct Entry {
    std::string name;
    int dtype;
    std::vector<int64_t> shape;
    size_t begin, end;   // relative to the data section
    int64_t numel() const {
        int64_t n = 1;
        for (int64_t d : shape) n *= d;
        return n;
    }
};

class Shard {
  public:
    explicit Shard(const std::string& path) : path_(path) {
        fd_ = ::open(path.c_str(), O_RDONLY);
        if (fd_ < 0) throw Error("safetensors: cannot open " + path);
        struct stat sb {};
        if (::fstat(fd_, &sb) != 0) throw Error("safetensors: cannot stat " + path);
        size_ = static_cast<size_t>(sb.st_size);
        if (size_ < 8) throw Error("safetensors: " + path + " is shorter than its 8-byte header length");
        base_ = ::mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0);
        if (base_ == MAP_FAILED) {
            base_ = nullptr;
            throw Error("safetensors: cannot map " + path);
        }
        uint64_t hlen = 0;
        std::memcpy(&hlen, base_, 8);   // little-endian on every host this builds for
        if (hlen == 0 || hlen > size_ - 8) {
            throw Error("safetensors: " + path + ": header length " + std::to_string(hlen) +
                        " does not fit in a file of " + std::to_string(size_) + " bytes");
        }
        data_ = 8 + static_cast<size_t>(hlen);
        const Json doc = JsonReader(static_cast<const char*>(base_) + 8, hlen).document();
        if (doc.kind != Json::OBJ) throw Error("safetensors: " + path + ": header is not a JSON object");
        for (const auto& kv : doc.obj) {
            if (kv.first == "__metadata__") continue;
            entries_.push_back(entry(kv.first, kv.second));
        }
        std::sort(entries_.begin(), entries_.end(),
                  [](const Entry& a, const Entry& b) { return a.name < b.name; });
        for (size_t k = 1; k < entries_.size(); ++k)
            if (entries_[k].name == entries_[k - 1].name)
                throw Error("safetensors: " + path + " names tensor '" + entries_[k].name + "' twice");
    }
    ~Shard() {
        if (base_) ::munmap(base_, size_);
        if (fd_ >= 0) ::close(fd_);
    }
    Shard(const Shard&) = delete;
    Shard& operator=(const Shard&) = delete;

    const std::vector<Entry>& entries() const { return entries_; }
    const std::string& path() const { return path_; }
    size_t bytes() const { return size_; }

    const Entry* find(const std::string& name) const {
        auto it = std::lower_bound(entries_.begin(), entries_.end(), name,
                                   [](const Entry& e, const std::string& n) { return e.name < n; });
        return it != entries_.end() && it->name == name ? &*it : nullptr;
    }
    const char* data(const Entry& e) const { return static_cast<const char*>(base_) + data_ + e.begin; }

    // Up to five names that contain `name` or are contained in it, in name order.
    std::vector<std::string> near(const std::string& name) const {
        std::vector<std::string> out;
        for (const auto& e : entries_) {
            if (e.name.find(name) != std::string::npos || name.find(e.name) != std::string::npos) {
                out.push_back(e.name);
                if (out.size() == 5) break;
            }
        }
        return out;
    }

  private:
    std::string path_;
    int fd_ = -1;
    void* base_ = nullptr;
    size_t size_ = 0, data_ = 0;
    std::vector<Entry> entries_;

    Entry entry(const std::string& name, const Json& v) const {
        const auto field = [&](const char* key, Json::Kind kind) -> const Json& {
            const Json* f = v.kind == Json::OBJ ? v.find(key) : nullptr;
            if (!f || f->kind != kind)
                throw Error("safetensors: " + path_ + ": tensor '" + name + "' has no valid '" + key + "'");
            return *f;
        };
        const auto ints = [&](const Json& a, const char* key) {
            std::vector<int64_t> out;
            for (const Json& x : a.arr) {
                if (x.kind != Json::NUM || x.num < 0 || x.num != std::floor(x.num) || x.num > 9.0e15)
                    throw Error("safetensors: " + path_ + ": tensor '" + name + "': '" + key +
                                "' holds something other than a non-negative integer");
                out.push_back(static_cast<int64_t>(x.num));
            }
            return out;
        };
        Entry e;
        e.name = name;
        e.dtype = st_dtype_parse(field("dtype", Json::STR).str, name);
        e.shape = ints(field("shape", Json::ARR), "shape");
        const std::vector<int64_t> off = ints(field("data_offsets", Json::ARR), "data_offsets");
        if (off.size() != 2) throw Error("safetensors: " + path_ + ": tensor '" + name + "' needs two data_offsets");
        e.begin = static_cast<size_t>(off[0]);
        e.end = static_cast<size_t>(off[1]);
        double want = st_dtype_bytes(e.dtype);
        for (int64_t d : e.shape) want *= static_cast<double>(d);
        if (e.end < e.begin || static_cast<double>(e.end - e.begin) != want) {
            throw Error("safetensors: " + path_ + ": tensor '" + name + "' spans " +
                        std::to_string(static_cast<long long>(e.end) - static_cast<long long>(e.begin)) +
                        " bytes but its shape and dtype need " + std::to_string(static_cast<long long>(want)));
        }
        if (e.end > size_ - data_) {
            throw Error("safetensors: " + path_ + ": tensor '" + name + "' runs past the end of the file");
        }
        return e;
    }
};

// ---- conversion ---------------------------------------------------------------------------

// [b, e) of `n` elements of `src` (dtype `st`) into `dst` as `target` (BH_BF16 or BH_F32).
void convert_range(const char* src, int st, void* dst, int target, int64_t b, int64_t e) {
    if (target == BH_BF16) {
        bf16_t* out = static_cast<bf16_t*>(dst);
        if (st == ST_BF16) {
            std::memcpy(out + b, src + 2 * b, static_cast<size_t>(e - b) * 2);
        } else {   // ST_F32 (the only other dtype that converts)
            for (int64_t i = b; i < e; ++i) {
                float f;
                std::memcpy(&f, src + 4 * i, 4);
                out[i] = f2bf(f);
            }
        }
    } else {
        float* out = static_cast<float*>(dst);
        if (st == ST_F32) {
            std::memcpy(out + b, src + 4 * b, static_cast<size_t>(e - b) * 4);
        } else {
            for (int64_t i = b; i < e; ++i) {
                bf16_t h;
                std::memcpy(&h, src + 2 * i, 2);
                out[i] = bf2f(h);
            }
        }
    }
}

// Converts `n` elements; large ranges are split over the host's cores (every element goes
// through the same function whichever thread holds it, so the bytes do not depend on the split).
void convert(const char* src, int st, void* dst, int target, int64_t n, const std::string& name) {
    if (st == ST_F16 || st == ST_F8_E4M3) {
        throw Error(std::string("weights: '") + name + "' is " + st_dtype_name(st) +
                    ", which has no per-element conversion to the compute dtype here (as in the "
                    "reference runtime); convert the checkpoint to F32 or BF16 deliberately");
    }
    if (target != BH_BF16 && target != BH_F32) throw Error("weights: target dtype must be bf16 or fp32");
    const int64_t min_chunk = int64_t{1} << 21;
    const int64_t threads = std::max<int64_t>(
        1, std::min<int64_t>(std::thread::hardware_concurrency(), n / min_chunk));
    if (threads == 1) {
        convert_range(src, st, dst, target, 0, n);
        return;
    }
    std::vector<std::thread> pool;
    const int64_t chunk = (n + threads - 1) / threads;
    for (int64_t t = 0; t < threads; ++t) {
        const int64_t b = t * chunk, e = std::min(n, b + chunk);
        if (b < e) pool.emplace_back(convert_range, src, st, dst, target, b, e);
    }
    for (auto& th : pool) th.join();
}

}  // namespace

// ---- a checkpoint component (several shards) ---------------------------------------------

struct Checkpoint {
    std::vector<std::unique_ptr<Shard>> shards;

    const Shard* holder(const std::string& name, const Entry** e) const {
        for (const auto& s : shards) {
            if (const Entry* f = s->find(name)) {
                *e = f;
                return s.get();
            }
        }
        return nullptr;
    }

    // The entry for `name`, or an error naming the near misses (the first shard's, as in the
    // reference's CheckpointWeights::get).
    const Shard* require(const std::string& name, const Entry** e) const {
        if (const Shard* s = holder(name, e)) return s;
        std::string msg = "weights: '" + name + "' is missing from " + shards.front()->path() +
                          (shards.size() > 1 ? " and the other shards" : "") +
                          ". A model run with a missing weight would produce a plausible image "
                          "from wrong numbers, so this is fatal, never a zero-fill";
        const std::vector<std::string> near = shards.front()->near(name);
        if (!near.empty()) {
            msg += ". Did you mean: ";
            for (size_t k = 0; k < near.size(); ++k) msg += (k ? ", " : "") + near[k];
        }
        throw Error(msg);
    }
};

}  // namespace bh

struct bh_checkpoint : bh::Checkpoint {};

// ---- the DiT's weights on the device -------------------------------------------------------

struct bh_dit_device_weights {
    void* arena = nullptr;
    int64_t bytes = 0;
    bh_dit_weights view{};
    std::vector<bh_dit_block_weights> blocks;
    ~bh_dit_device_weights() {
        if (arena) (void)hipFree(arena);
    }
};

struct bh_t5_device_weights {
    void* arena = nullptr;
    int64_t bytes = 0;
    std::vector<std::string> names;
    std::vector<const char*> cnames;
    std::vector<const void*> ptrs;
    bh_t5_weights view{};
    ~bh_t5_device_weights() {
        if (arena) (void)hipFree(arena);
    }
};

struct bh_vae_device_weights {
    void* arena = nullptr;
    int64_t bytes = 0;
    std::vector<std::string> names;
    std::vector<const char*> cnames;
    std::vector<const void*> ptrs;
    bh_vae_weights view{};
    ~bh_vae_device_weights() {
        if (arena) (void)hipFree(arena);
    }
};

namespace bh {
namespace {

// One DiT tensor: its checkpoint name, the shape the configuration implies, and the struct
// field that receives its device address (declare_pixart_shapes, weights.cpp:246-282).
struct Want {
    std::string name;
    std::vector<int64_t> shape;
    const void** slot;
};

std::string shape_str(const std::vector<int64_t>& s) {
    std::string out = "[";
    for (size_t k = 0; k < s.size(); ++k) out += (k ? ", " : "") + std::to_string(s[k]);
    return out + "]";
}

std::vector<Want> dit_tensors(const bh_dit_config& c, bh_dit_device_weights& w) {
    const int64_t d = static_cast<int64_t>(c.num_heads) * c.head_dim;
    const int64_t dff = static_cast<int64_t>(std::llround(static_cast<double>(d) * c.mlp_ratio));
    const int64_t p = c.patch_size;
    bh_dit_weights& t = w.view;
    std::vector<Want> out = {
        {"pos_embed.proj.weight", {d, c.in_channels, p, p}, &t.pos_embed_w},
        {"pos_embed.proj.bias", {d}, &t.pos_embed_b},
        {"adaln_single.emb.timestep_embedder.linear_1.weight", {d, 256}, &t.t_emb1_w},
        {"adaln_single.emb.timestep_embedder.linear_1.bias", {d}, &t.t_emb1_b},
        {"adaln_single.emb.timestep_embedder.linear_2.weight", {d, d}, &t.t_emb2_w},
        {"adaln_single.emb.timestep_embedder.linear_2.bias", {d}, &t.t_emb2_b},
        {"adaln_single.linear.weight", {6 * d, d}, &t.adaln_w},
        {"adaln_single.linear.bias", {6 * d}, &t.adaln_b},
        {"caption_projection.linear_1.weight", {d, c.caption_channels}, &t.cap1_w},
        {"caption_projection.linear_1.bias", {d}, &t.cap1_b},
        {"caption_projection.linear_2.weight", {d, d}, &t.cap2_w},
        {"caption_projection.linear_2.bias", {d}, &t.cap2_b},
        {"scale_shift_table", {2, d}, &t.out_table},
        {"proj_out.weight", {p * p * c.out_channels, d}, &t.proj_out_w},
        {"proj_out.bias", {p * p * c.out_channels}, &t.proj_out_b},
    };
    // The arena keeps this order (each tensor 256-byte aligned): a layer's self-attention Q, K
    // and V weights back to back, then their biases, and every layer's cross-attention K and V
    // weights back to back in layer order after all other layer tensors, then their biases. The
    // fused dit-step engine then reads the packed [3d, d] and [L * 2d, d] projections in place
    // instead of copying them (when d * 2 bytes is a multiple of the alignment, as at d = 1152).
    const auto pre = [](int i) { return "transformer_blocks." + std::to_string(i) + "."; };
    for (int i = 0; i < c.num_layers; ++i) {
        bh_dit_block_weights& b = w.blocks[static_cast<size_t>(i)];
        const auto add = [&](const char* n, std::vector<int64_t> s, const void** slot) {
            out.push_back({pre(i) + n, std::move(s), slot});
        };
        add("scale_shift_table", {6, d}, &b.scale_shift_table);
        add("attn1.to_q.weight", {d, d}, &b.attn1_q_w);
        add("attn1.to_k.weight", {d, d}, &b.attn1_k_w);
        add("attn1.to_v.weight", {d, d}, &b.attn1_v_w);
        add("attn1.to_q.bias", {d}, &b.attn1_q_b);
        add("attn1.to_k.bias", {d}, &b.attn1_k_b);
        add("attn1.to_v.bias", {d}, &b.attn1_v_b);
        add("attn1.to_out.0.weight", {d, d}, &b.attn1_o_w); add("attn1.to_out.0.bias", {d}, &b.attn1_o_b);
        add("attn2.to_q.weight", {d, d}, &b.attn2_q_w); add("attn2.to_q.bias", {d}, &b.attn2_q_b);
        add("attn2.to_out.0.weight", {d, d}, &b.attn2_o_w); add("attn2.to_out.0.bias", {d}, &b.attn2_o_b);
        add("ff.net.0.proj.weight", {dff, d}, &b.ff0_w); add("ff.net.0.proj.bias", {dff}, &b.ff0_b);
        add("ff.net.2.weight", {d, dff}, &b.ff2_w); add("ff.net.2.bias", {d}, &b.ff2_b);
    }
    for (int i = 0; i < c.num_layers; ++i) {
        bh_dit_block_weights& b = w.blocks[static_cast<size_t>(i)];
        out.push_back({pre(i) + "attn2.to_k.weight", {d, d}, &b.attn2_k_w});
        out.push_back({pre(i) + "attn2.to_v.weight", {d, d}, &b.attn2_v_w});
    }
    for (int i = 0; i < c.num_layers; ++i) {
        bh_dit_block_weights& b = w.blocks[static_cast<size_t>(i)];
        out.push_back({pre(i) + "attn2.to_k.bias", {d}, &b.attn2_k_b});
        out.push_back({pre(i) + "attn2.to_v.bias", {d}, &b.attn2_v_b});
    }
    return out;
}

// A checkpoint shape matches when it is the expected one, or (for the patch embedding) its
// flattened [out, in*kh*kw] form, which holds the same bytes in the same order.
bool shape_ok(const std::string& name, const std::vector<int64_t>& got, const std::vector<int64_t>& want) {
    if (got == want) return true;
    if (name == "pos_embed.proj.weight" && got.size() == 2 && want.size() == 4)
        return got[0] == want[0] && got[1] == want[1] * want[2] * want[3];
    return false;
}

constexpr int64_t kAlign = 256;
constexpr int64_t kStageBytes = int64_t{32} << 20;   // two halves of 16 MiB

struct PinnedStage {
    char* p = nullptr;
    hipEvent_t done[2] = {nullptr, nullptr};
    PinnedStage() {
        hip_check(hipHostMalloc(reinterpret_cast<void**>(&p), kStageBytes, hipHostMallocDefault),
                  "hipHostMalloc (weight staging)");
        for (auto& e : done) hip_check(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreate");
    }
    ~PinnedStage() {   // no copy may still read the staging when it is freed (an error path)
        for (auto& e : done) {
            if (!e) continue;
            (void)hipEventSynchronize(e);
            (void)hipEventDestroy(e);
        }
        if (p) (void)hipHostFree(p);
    }
};

}  // namespace

// Checks every wanted tensor (present, shape, F32 or BF16) before allocating anything, then
// converts each to bf16 on the host into page-locked staging and copies it into one device arena
// on `st`, setting *want[i].slot to its address. Returns the arena's size; *arena owns it.
int64_t upload_arena(const Checkpoint& ck, const std::vector<Want>& want, hipStream_t st, void** arena) {
    struct Src { const Shard* shard; const Entry* entry; int64_t offset; };
    std::vector<Src> src;
    int64_t total = 0;
    for (const Want& t : want) {
        const Entry* e = nullptr;
        const Shard* s = ck.require(t.name, &e);
        if (!shape_ok(t.name, e->shape, t.shape)) {
            throw Error("weights: '" + t.name + "' is " + shape_str(e->shape) +
                        " in the checkpoint, but this configuration needs " + shape_str(t.shape));
        }
        if (e->dtype != ST_F32 && e->dtype != ST_BF16) {
            throw Error(std::string("weights: '") + t.name + "' is " + st_dtype_name(e->dtype) +
                        ", which has no per-element conversion to bf16 here (as in the reference "
                        "runtime); convert the checkpoint to F32 or BF16 deliberately");
        }
        src.push_back({s, e, total});
        total += (e->numel() * 2 + kAlign - 1) / kAlign * kAlign;
    }
    hip_check(hipMalloc(arena, static_cast<size_t>(std::max<int64_t>(total, kAlign))), "hipMalloc (weights)");
    PinnedStage stage;
    const int64_t half = kStageBytes / 2;
    int buf = 0;
    bool used[2] = {false, false};
    for (size_t k = 0; k < want.size(); ++k) {
        char* dev = static_cast<char*>(*arena) + src[k].offset;
        *want[k].slot = dev;
        const Entry& e = *src[k].entry;
        const char* host = src[k].shard->data(e);
        const int64_t n = e.numel();
        const int64_t per = half / 2;   // bf16 elements per staging half
        for (int64_t b = 0; b < n; b += per) {
            const int64_t m = std::min(per, n - b);
            if (used[buf]) hip_check(hipEventSynchronize(stage.done[buf]), "hipEventSynchronize");
            char* h = stage.p + buf * half;
            convert(host + b * st_dtype_bytes(e.dtype), e.dtype, h, BH_BF16, m, e.name);
            hip_check(hipMemcpyAsync(dev + 2 * b, h, static_cast<size_t>(m) * 2, hipMemcpyHostToDevice, st),
                      "hipMemcpyAsync (weights)");
            hip_check(hipEventRecord(stage.done[buf], st), "hipEventRecord");
            used[buf] = true;
            buf ^= 1;
        }
    }
    hip_check(hipStreamSynchronize(st), "hipStreamSynchronize (weights)");
    return total;
}

}  // namespace bh

extern "C" {

int bh_checkpoint_open(const char* const* shard_paths, int n_shards, bh_checkpoint** out) {
    return bh::guarded([&] {
        bh::require(out != nullptr, "checkpoint_open: null output handle");
        *out = nullptr;
        bh::require(n_shards > 0 && shard_paths != nullptr, "checkpoint_open: no shards given");
        auto ck = std::make_unique<bh_checkpoint>();
        for (int k = 0; k < n_shards; ++k) {
            bh::require(shard_paths[k] != nullptr, "checkpoint_open: null shard path");
            ck->shards.push_back(std::make_unique<bh::Shard>(shard_paths[k]));
        }
        *out = ck.release();
    });
}

int bh_checkpoint_open_component(const char* dir, const char* component, bh_checkpoint** out) {
    return bh::guarded([&] {
        bh::require(out != nullptr, "checkpoint_open_component: null output handle");
        *out = nullptr;
        bh::require(dir && component, "checkpoint_open_component: null directory or component");
        const std::string root = std::string(dir) + "/" + component;
        DIR* dp = ::opendir(root.c_str());
        if (!dp) {
            throw bh::Error("weights: no directory " + root + ". A checkpoint is read in the "
                            "published layout (transformer/, vae/, text_encoder/), one directory "
                            "per component");
        }
        std::vector<std::string> shards;
        while (const dirent* ent = ::readdir(dp)) {
            const std::string n = ent->d_name;
            const std::string ext = ".safetensors";
            if (n.size() > ext.size() && n.compare(n.size() - ext.size(), ext.size(), ext) == 0) {
                struct stat sb {};
                const std::string path = root + "/" + n;
                if (::stat(path.c_str(), &sb) == 0 && S_ISREG(sb.st_mode)) shards.push_back(path);
            }
        }
        ::closedir(dp);
        std::sort(shards.begin(), shards.end());
        if (shards.empty()) throw bh::Error("weights: no .safetensors under " + root);
        auto ck = std::make_unique<bh_checkpoint>();
        for (const auto& p : shards) ck->shards.push_back(std::make_unique<bh::Shard>(p));
        *out = ck.release();
    });
}

void bh_checkpoint_close(bh_checkpoint* ck) { delete ck; }

int64_t bh_checkpoint_count(const bh_checkpoint* ck) {
    if (!ck) return -1;
    int64_t n = 0;
    for (const auto& s : ck->shards) n += static_cast<int64_t>(s->entries().size());
    return n;
}

int bh_checkpoint_entry(const bh_checkpoint* ck, int64_t index, const char** name, int* dtype,
                        int* rank, int64_t* shape, int max_rank) {
    return bh::guarded([&] {
        bh::require(ck != nullptr, "checkpoint_entry: null handle");
        int64_t i = index;
        for (const auto& s : ck->shards) {
            const auto& es = s->entries();
            if (i >= 0 && i < static_cast<int64_t>(es.size())) {
                const bh::Entry& e = es[static_cast<size_t>(i)];
                if (name) *name = e.name.c_str();
                if (dtype) *dtype = e.dtype;
                if (rank) *rank = static_cast<int>(e.shape.size());
                if (shape) {
                    bh::require(static_cast<int>(e.shape.size()) <= max_rank,
                                "checkpoint_entry: '" + e.name + "' has rank " +
                                    std::to_string(e.shape.size()) + ", above max_rank");
                    for (size_t k = 0; k < e.shape.size(); ++k) shape[k] = e.shape[k];
                }
                return;
            }
            i -= static_cast<int64_t>(es.size());
        }
        throw bh::Error("checkpoint_entry: index " + std::to_string(index) + " out of range");
    });
}

int bh_checkpoint_find(const bh_checkpoint* ck, const char* name, int* dtype, int* rank,
                       int64_t* shape, int max_rank) {
    return bh::guarded([&] {
        bh::require(ck != nullptr && name != nullptr, "checkpoint_find: null handle or name");
        const bh::Entry* e = nullptr;
        ck->require(name, &e);
        if (dtype) *dtype = e->dtype;
        if (rank) *rank = static_cast<int>(e->shape.size());
        if (shape) {
            bh::require(static_cast<int>(e->shape.size()) <= max_rank,
                        std::string("checkpoint_find: '") + name + "' has a rank above max_rank");
            for (size_t k = 0; k < e->shape.size(); ++k) shape[k] = e->shape[k];
        }
    });
}

int bh_checkpoint_read(const bh_checkpoint* ck, const char* name, int dtype, void* dst,
                       int64_t numel) {
    return bh::guarded([&] {
        bh::require(ck != nullptr && name != nullptr, "checkpoint_read: null handle or name");
        const bh::Entry* e = nullptr;
        const bh::Shard* s = ck->require(name, &e);
        bh::require(numel == e->numel(), std::string("checkpoint_read: '") + name + "' holds " +
                                             std::to_string(e->numel()) + " elements, not " +
                                             std::to_string(numel));
        bh::require(dst != nullptr || numel == 0, "checkpoint_read: null destination");
        bh::convert(s->data(*e), e->dtype, dst, dtype, numel, name);
    });
}

int bh_dit_weights_load(const bh_checkpoint* ck, const bh_dit_config* cfg, void* stream,
                        bh_dit_device_weights** out) {
    return bh::guarded([&] {
        bh::require(out != nullptr, "dit_weights_load: null output handle");
        *out = nullptr;
        bh::require(ck != nullptr && cfg != nullptr, "dit_weights_load: null checkpoint or config");
        bh::require(cfg->num_layers > 0 && cfg->num_heads > 0 && cfg->head_dim > 0 &&
                        cfg->patch_size > 0 && cfg->in_channels > 0 && cfg->out_channels > 0 &&
                        cfg->caption_channels > 0 && cfg->mlp_ratio > 0,
                    "dit_weights_load: the configuration has a non-positive size");
        auto w = std::make_unique<bh_dit_device_weights>();
        w->blocks.resize(static_cast<size_t>(cfg->num_layers));
        const std::vector<bh::Want> want = bh::dit_tensors(*cfg, *w);
        w->bytes = bh::upload_arena(*ck, want, static_cast<hipStream_t>(stream), &w->arena);
        w->view.blocks = w->blocks.data();
        *out = w.release();
    });
}

int bh_vae_weights_load(const bh_checkpoint* ck, const bh_vae_config* cfg, void* stream,
                        bh_vae_device_weights** out) {
    return bh::guarded([&] {
        bh::require(out != nullptr, "vae_weights_load: null output handle");
        *out = nullptr;
        bh::require(ck != nullptr && cfg != nullptr, "vae_weights_load: null checkpoint or config");
        bh::require(cfg->num_blocks >= 1 && cfg->num_blocks <= 8 && cfg->layers_per_block >= 0 &&
                        cfg->latent_channels > 0,
                    "vae_weights_load: configuration out of range");
        auto w = std::make_unique<bh_vae_device_weights>();
        const auto table = bh::vae_tensor_shapes(*cfg);
        w->names.reserve(table.size());
        w->ptrs.assign(table.size(), nullptr);
        std::vector<bh::Want> want;
        for (size_t i = 0; i < table.size(); ++i) {
            w->names.push_back(table[i].first);
            want.push_back({table[i].first, table[i].second, &w->ptrs[i]});
        }
        w->bytes = bh::upload_arena(*ck, want, static_cast<hipStream_t>(stream), &w->arena);
        for (const auto& n : w->names) w->cnames.push_back(n.c_str());
        w->view.count = static_cast<int>(w->names.size());
        w->view.names = w->cnames.data();
        w->view.tensors = w->ptrs.data();
        *out = w.release();
    });
}

int bh_t5_weights_load(const bh_checkpoint* ck, const bh_t5_config* cfg, void* stream,
                       bh_t5_device_weights** out) {
    return bh::guarded([&] {
        bh::require(out != nullptr, "t5_weights_load: null output handle");
        *out = nullptr;
        bh::require(ck != nullptr && cfg != nullptr, "t5_weights_load: null checkpoint or config");
        bh::require(cfg->num_layers >= 0 && cfg->d_model > 0 && cfg->d_ff > 0 && cfg->d_kv > 0 &&
                        cfg->num_heads > 0 && cfg->vocab_size > 0 && cfg->num_buckets > 0,
                    "t5_weights_load: configuration out of range");
        auto w = std::make_unique<bh_t5_device_weights>();
        const auto table = bh::t5_tensor_shapes(*cfg);
        w->names.reserve(table.size());
        w->ptrs.assign(table.size(), nullptr);
        std::vector<bh::Want> want;
        for (size_t i = 0; i < table.size(); ++i) {
            w->names.push_back(table[i].first);
            want.push_back({table[i].first, table[i].second, &w->ptrs[i]});
        }
        w->bytes = bh::upload_arena(*ck, want, static_cast<hipStream_t>(stream), &w->arena);
        for (const auto& n : w->names) w->cnames.push_back(n.c_str());
        w->view.count = static_cast<int>(w->names.size());
        w->view.names = w->cnames.data();
        w->view.tensors = w->ptrs.data();
        *out = w.release();
    });
}

const bh_t5_weights* bh_t5_weights_view(const bh_t5_device_weights* w) { return w ? &w->view : nullptr; }

int64_t bh_t5_weights_bytes(const bh_t5_device_weights* w) { return w ? w->bytes : -1; }

void bh_t5_weights_free(bh_t5_device_weights* w) { delete w; }

const bh_vae_weights* bh_vae_weights_view(const bh_vae_device_weights* w) { return w ? &w->view : nullptr; }

int64_t bh_vae_weights_bytes(const bh_vae_device_weights* w) { return w ? w->bytes : -1; }

void bh_vae_weights_free(bh_vae_device_weights* w) { delete w; }

const bh_dit_weights* bh_dit_weights_view(const bh_dit_device_weights* w) {
    return w ? &w->view : nullptr;
}

int64_t bh_dit_weights_bytes(const bh_dit_device_weights* w) { return w ? w->bytes : -1; }

void bh_dit_weights_free(bh_dit_device_weights* w) { delete w; }

}  // extern "C"
