// moepack.cpp — the MoEPack install reader in front of the HBM-resident expert
// path. It parses manifest.json and packed_experts/layout.json and validates
// them with the reference's rules. It also derives the routed-expert sub-tensor
// offsets, and uploads a layer file into one HBM image with each expert blob at
// its LOGICAL position (the kernels address expert e at base + e * stride).
//
//   MoEPackManifestCodec.validate        MoEPackManifestV1.swift:378-478
//   linear-attention / vision / draft    MoEPackManifestV1.swift:497-640
//   ManifestReader.decode / validate     ManifestReader.swift:182-245
//   validateQuant                        ManifestReader.swift:250-313
//   MoEPackV1StructuralValidator         MoEPackPackedExpertsLayoutV1.swift:84-212
//   PackedExpertsLayoutReader.decode     PackedExpertsLayout.swift:83-115
//   routedExpertOffsets / physical       ModelExpertIO.swift:56-88
//   MoEPackModelDirectory (openat walk)  MoEPackModelDirectory.swift:9-115
//   MoEPackPathValidator                 MoEPackFormatV1.swift:86-111
//
// Host code only. Errors carry the reference's ModelError case name at the
// start of the message (indexCorrupt, notAMoEPackDirectory, unsupportedVersion,
// unknownFlag, expertStrideNotPageAligned, missingFile, partialInstall,
// posixFailed). Content errors return TSG_ERR_FORMAT and file-system errors
// TSG_ERR_IO.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <utility>
#include <vector>

#include "../../include/tsugumi_hip.h"

namespace tsg {
tsg_status fail(tsg_status status, const char* fmt, ...);
void layer_geometry(const tsg_layer* layer, int* device, uint32_t* num_experts,
                    uint64_t* expert_stride, tsg_expert_offsets* offsets);
}

namespace {

constexpr uint64_t kAlignmentBytes = 16384;                       // MoEPackFormatV1.alignmentBytes
constexpr uint64_t kManifestMaxBytes = 4ull * 1024 * 1024;        // ManifestReader.defaultMaxBytes
constexpr uint64_t kLayoutMaxBytes = 64ull * 1024 * 1024;         // packedExpertsLayoutMaxBytes
constexpr int kVersionMajor = 1;
constexpr int kVersionMinorVision = 1;
constexpr int kVersionMinorDraft = 2;
constexpr int kVersionMinorLinearAttention = 3;
constexpr int kMaxJsonDepth = 64;
constexpr uint64_t kStagingBytes = 64ull * 1024 * 1024;           // per staging buffer

struct LoadError {
    tsg_status status;
    std::string message;
};

[[noreturn]] void throw_error(tsg_status status, std::string message) {
    throw LoadError{status, std::move(message)};
}
[[noreturn]] void corrupt(const std::string& detail) {
    throw_error(TSG_ERR_FORMAT, "indexCorrupt: " + detail);
}

// ------------------------------------------------------------------ JSON ----
// RFC 8259 reader. Numbers keep their literal text so 64-bit offsets convert
// exactly. Duplicate object keys are rejected (a reader that kept either copy
// would disagree with some other reader about the install).

struct JVal {
    enum Kind : uint8_t { Null, Bool, Num, Str, Arr, Obj };
    Kind kind = Null;
    bool boolean = false;
    std::string text;                 // a string's contents or a number's literal
    std::vector<std::string> keys;    // object member names, document order
    std::vector<JVal> items;          // array elements or object member values

    const JVal* find(const char* key) const {
        for (size_t i = 0; i < keys.size(); ++i)
            if (keys[i] == key) return &items[i];
        return nullptr;
    }
};

bool utf8_valid(const unsigned char* s, size_t n) {
    size_t i = 0;
    while (i < n) {
        const unsigned c = s[i];
        if (c < 0x80) { ++i; continue; }
        int len;
        uint32_t cp;
        if ((c & 0xE0) == 0xC0) { len = 2; cp = c & 0x1F; }
        else if ((c & 0xF0) == 0xE0) { len = 3; cp = c & 0x0F; }
        else if ((c & 0xF8) == 0xF0) { len = 4; cp = c & 0x07; }
        else return false;
        if (i + len > n) return false;
        for (int k = 1; k < len; ++k) {
            if ((s[i + k] & 0xC0) != 0x80) return false;
            cp = (cp << 6) | (s[i + k] & 0x3F);
        }
        if ((len == 2 && cp < 0x80) || (len == 3 && cp < 0x800) || (len == 4 && cp < 0x10000) ||
            cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF))
            return false;
        i += len;
    }
    return true;
}

class JsonReader {
public:
    JsonReader(const char* data, size_t n, const char* doc) : p_(data), begin_(data), end_(data + n), doc_(doc) {}

    void parse(JVal& root) {
        if (!utf8_valid(reinterpret_cast<const unsigned char*>(begin_), end_ - begin_))
            corrupt(std::string(doc_) + ": not valid UTF-8");
        skip_ws();
        value(root, 0);
        skip_ws();
        if (p_ != end_) error("trailing characters after the document");
    }

private:
    const char* p_;
    const char* begin_;
    const char* end_;
    const char* doc_;

    [[noreturn]] void error(const char* what) {
        char buf[64];
        snprintf(buf, sizeof buf, " at byte %zu", (size_t)(p_ - begin_));
        corrupt(std::string(doc_) + ": " + what + buf);
    }
    void skip_ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool literal(const char* word) {
        const size_t n = strlen(word);
        if ((size_t)(end_ - p_) < n || memcmp(p_, word, n) != 0) return false;
        p_ += n;
        return true;
    }

    void value(JVal& v, int depth) {
        if (depth > kMaxJsonDepth) error("nesting too deep");
        if (p_ >= end_) error("unexpected end of input");
        const char c = *p_;
        if (c == '{') return object(v, depth);
        if (c == '[') return array(v, depth);
        if (c == '"') { v.kind = JVal::Str; return string(v.text); }
        if (c == '-' || (c >= '0' && c <= '9')) return number(v);
        if (literal("true")) { v.kind = JVal::Bool; v.boolean = true; return; }
        if (literal("false")) { v.kind = JVal::Bool; v.boolean = false; return; }
        if (literal("null")) { v.kind = JVal::Null; return; }
        error("unexpected character");
    }

    void object(JVal& v, int depth) {
        v.kind = JVal::Obj;
        ++p_;
        skip_ws();
        if (p_ < end_ && *p_ == '}') { ++p_; return; }
        std::unordered_set<std::string> seen;
        for (;;) {
            skip_ws();
            if (p_ >= end_ || *p_ != '"') error("expected a member name");
            std::string key;
            string(key);
            if (v.keys.size() < 16) {
                for (const auto& k : v.keys)
                    if (k == key) error(("duplicate key \"" + key + "\"").c_str());
            } else {
                if (seen.empty()) seen.insert(v.keys.begin(), v.keys.end());
                if (!seen.insert(key).second) error(("duplicate key \"" + key + "\"").c_str());
            }
            skip_ws();
            if (p_ >= end_ || *p_ != ':') error("expected ':'");
            ++p_;
            skip_ws();
            v.keys.push_back(std::move(key));
            v.items.emplace_back();
            value(v.items.back(), depth + 1);
            skip_ws();
            if (p_ < end_ && *p_ == ',') { ++p_; continue; }
            if (p_ < end_ && *p_ == '}') { ++p_; return; }
            error("expected ',' or '}'");
        }
    }

    void array(JVal& v, int depth) {
        v.kind = JVal::Arr;
        ++p_;
        skip_ws();
        if (p_ < end_ && *p_ == ']') { ++p_; return; }
        for (;;) {
            skip_ws();
            v.items.emplace_back();
            value(v.items.back(), depth + 1);
            skip_ws();
            if (p_ < end_ && *p_ == ',') { ++p_; continue; }
            if (p_ < end_ && *p_ == ']') { ++p_; return; }
            error("expected ',' or ']'");
        }
    }

    unsigned hex4() {
        if (end_ - p_ < 4) error("truncated \\u escape");
        unsigned u = 0;
        for (int k = 0; k < 4; ++k) {
            const char h = *p_++;
            u <<= 4;
            if (h >= '0' && h <= '9') u |= h - '0';
            else if (h >= 'a' && h <= 'f') u |= h - 'a' + 10;
            else if (h >= 'A' && h <= 'F') u |= h - 'A' + 10;
            else error("bad \\u escape");
        }
        return u;
    }

    static void put_utf8(std::string& out, uint32_t cp) {
        if (cp < 0x80) {
            out += (char)cp;
        } else if (cp < 0x800) {
            out += (char)(0xC0 | (cp >> 6));
            out += (char)(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            out += (char)(0xE0 | (cp >> 12));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
        } else {
            out += (char)(0xF0 | (cp >> 18));
            out += (char)(0x80 | ((cp >> 12) & 0x3F));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
        }
    }

    void string(std::string& out) {
        ++p_;  // opening quote
        for (;;) {
            if (p_ >= end_) error("unterminated string");
            const unsigned char c = (unsigned char)*p_++;
            if (c == '"') return;
            if (c < 0x20) error("control character in string");
            if (c != '\\') { out += (char)c; continue; }
            if (p_ >= end_) error("unterminated escape");
            const char e = *p_++;
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
                    if (cp >= 0xD800 && cp <= 0xDBFF) {
                        if (end_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u') error("lone surrogate");
                        p_ += 2;
                        const uint32_t lo = hex4();
                        if (lo < 0xDC00 || lo > 0xDFFF) error("bad surrogate pair");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    } else if (cp >= 0xDC00 && cp <= 0xDFFF) {
                        error("lone surrogate");
                    }
                    put_utf8(out, cp);
                    break;
                }
                default: error("bad escape");
            }
        }
    }

    void number(JVal& v) {
        const char* s = p_;
        if (*p_ == '-') ++p_;
        if (p_ >= end_) error("bad number");
        if (*p_ == '0') {
            ++p_;
        } else if (*p_ >= '1' && *p_ <= '9') {
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        } else {
            error("bad number");
        }
        if (p_ < end_ && *p_ == '.') {
            ++p_;
            if (p_ >= end_ || *p_ < '0' || *p_ > '9') error("bad fraction");
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
            ++p_;
            if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
            if (p_ >= end_ || *p_ < '0' || *p_ > '9') error("bad exponent");
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        v.kind = JVal::Num;
        v.text.assign(s, p_);
    }
};

// Typed access in the manner of Swift's Decodable: a missing key or a wrong
// type is a decode error naming the path; `null` reads as absent for
// optionals. Integer fields take integer literals only.
struct Decoder {
    std::string doc;

    [[noreturn]] void bad(const std::string& path, const char* what) const {
        corrupt(doc + ": " + path + ": " + what);
    }
    const JVal& req(const JVal& obj, const char* key, const std::string& path) const {
        const JVal* v = obj.find(key);
        if (!v || v->kind == JVal::Null) bad(path + "." + key, "required key is missing");
        return *v;
    }
    static const JVal* opt(const JVal& obj, const char* key) {
        const JVal* v = obj.find(key);
        return (v && v->kind != JVal::Null) ? v : nullptr;
    }
    const JVal& object(const JVal& v, const std::string& path) const {
        if (v.kind != JVal::Obj) bad(path, "expected an object");
        return v;
    }
    const JVal& array(const JVal& v, const std::string& path) const {
        if (v.kind != JVal::Arr) bad(path, "expected an array");
        return v;
    }
    bool boolean(const JVal& v, const std::string& path) const {
        if (v.kind != JVal::Bool) bad(path, "expected a Bool");
        return v.boolean;
    }
    const std::string& str(const JVal& v, const std::string& path) const {
        if (v.kind != JVal::Str) bad(path, "expected a String");
        return v.text;
    }
    double real(const JVal& v, const std::string& path) const {
        if (v.kind != JVal::Num) bad(path, "expected a number");
        const double d = strtod(v.text.c_str(), nullptr);
        if (!std::isfinite(d)) bad(path, "number out of range");
        return d;
    }
    int64_t integer(const JVal& v, const std::string& path) const {
        if (v.kind != JVal::Num || v.text.find_first_of(".eE") != std::string::npos)
            bad(path, "expected an integer");
        errno = 0;
        char* endp = nullptr;
        const long long x = strtoll(v.text.c_str(), &endp, 10);
        if (errno == ERANGE || *endp) bad(path, "integer out of range");
        return (int64_t)x;
    }
    uint64_t unsigned64(const JVal& v, const std::string& path) const {
        if (v.kind != JVal::Num || v.text.find_first_of(".eE") != std::string::npos ||
            v.text[0] == '-')
            bad(path, "expected a non-negative integer");
        errno = 0;
        char* endp = nullptr;
        const unsigned long long x = strtoull(v.text.c_str(), &endp, 10);
        if (errno == ERANGE || *endp) bad(path, "integer out of range");
        return (uint64_t)x;
    }
    int64_t req_int(const JVal& o, const char* k, const std::string& path) const {
        return integer(req(o, k, path), path + "." + k);
    }
    uint64_t req_u64(const JVal& o, const char* k, const std::string& path) const {
        return unsigned64(req(o, k, path), path + "." + k);
    }
    double req_real(const JVal& o, const char* k, const std::string& path) const {
        return real(req(o, k, path), path + "." + k);
    }
    bool req_bool(const JVal& o, const char* k, const std::string& path) const {
        return boolean(req(o, k, path), path + "." + k);
    }
    std::string req_str(const JVal& o, const char* k, const std::string& path) const {
        return str(req(o, k, path), path + "." + k);
    }
};

std::string lower_ascii(std::string s) {
    for (char& c : s)
        if (c >= 'A' && c <= 'Z') c = (char)(c - 'A' + 'a');
    return s;
}

// ----------------------------------------------------------------- paths ----

// MoEPackPathValidator.validateRelativePath (MoEPackFormatV1.swift:89-102).
void validate_relative_path(const std::string& path, const std::string& field) {
    if (path.empty() || path[0] == '/' || path.find('\0') != std::string::npos)
        corrupt(field + ": unsafe relative path");
    size_t start = 0;
    for (;;) {
        const size_t slash = path.find('/', start);
        const std::string comp = path.substr(start, slash == std::string::npos ? std::string::npos
                                                                            : slash - start);
        if (comp.empty() || comp == "." || comp == "..") corrupt(field + ": non-canonical path");
        if (slash == std::string::npos) break;
        start = slash + 1;
    }
}

// MoEPackPathValidator.validateBasename (MoEPackFormatV1.swift:105-110).
void validate_basename(const std::string& name, const std::string& field) {
    validate_relative_path(name, field);
    if (name.find('/') != std::string::npos) corrupt(field + ": expected basename");
}

// appleFilesystemKey folds case and Unicode normalisation so that names a
// case-insensitive file system would merge compare equal. This reader folds
// ASCII case; non-ASCII bytes compare as written.
std::string filesystem_key(const std::string& path) { return lower_ascii(path); }

// ------------------------------------------------------------- manifest ----

struct QuantSlot {
    int64_t weight_bits = 0, group_size = 0;
    std::string scheme, scale_type, bias_type;
};

struct FileEntry {
    uint64_t size = 0;
    std::string sha256;
};

struct Manifest {
    std::string magic;
    int64_t version_major = 0, version_minor = 0;
    std::vector<std::pair<std::string, bool>> flags;
    std::string model_id;
    // arch
    int64_t hidden = 0, ffn = 0, moe_inter = 0, heads = 0, kv_heads = 0, full_kv_heads = 0,
            head_dim = 0, full_head_dim = 0, vocab = 0, sliding_window = 0, arch_layers = 0,
            arch_experts = 0, top_k = 0;
    double softcap = 0, rope = 0, full_rope = 0, partial_rotary = 0;
    std::string activation;
    std::vector<int64_t> full_mask;
    bool has_family = false;
    std::string family;
    bool has_kinds = false;
    std::vector<std::string> kinds;
    bool has_linear = false;
    int64_t lin_key_heads = 0, lin_value_heads = 0, lin_key_dim = 0, lin_value_dim = 0,
            lin_conv = 0, lin_layers = 0;
    // quant
    bool has_quant = false;
    QuantSlot embedding, attention, router, shared_expert, routed_expert;
    // vision / draft: only the fields the file checks read
    bool has_vision = false, has_draft = false;
    std::string vision_path, draft_path;
    uint64_t vision_payload = 0, draft_payload = 0;
    std::vector<std::pair<std::string, FileEntry>> files;  // document order
    std::unordered_map<std::string, size_t> file_index;   // path -> files[]
    int64_t experts_per_layer = 0, num_layers = 0;
    uint64_t expert_stride = 0;

    bool flag(const char* name) const {
        for (const auto& f : flags)
            if (f.first == name) return f.second;
        return false;
    }
    const FileEntry* file(const std::string& path) const {
        auto it = file_index.find(path);
        return it == file_index.end() ? nullptr : &files[it->second].second;
    }
};

QuantSlot decode_slot(const Decoder& d, const JVal& q, const char* name) {
    const std::string path = std::string("manifest.quant.") + name;
    const JVal& s = d.object(d.req(q, name, "manifest.quant"), path);
    QuantSlot slot;
    slot.weight_bits = d.req_int(s, "weightBits", path);
    slot.scheme = d.req_str(s, "scheme", path);
    slot.scale_type = d.req_str(s, "scaleType", path);
    slot.bias_type = d.req_str(s, "biasType", path);
    slot.group_size = d.req_int(s, "groupSize", path);
    return slot;
}

// The wire structure (MoEPackManifestV1.swift:3-322): every non-optional key
// must be present with its type; unknown keys are ignored.
Manifest decode_manifest(const JVal& root) {
    Decoder d{"manifest.json"};
    Manifest m;
    const std::string R = "manifest";
    d.object(root, R);
    m.magic = d.req_str(root, "magic", R);
    m.version_major = d.req_int(root, "versionMajor", R);
    m.version_minor = d.req_int(root, "versionMinor", R);
    const JVal& flags = d.object(d.req(root, "flags", R), R + ".flags");
    for (size_t i = 0; i < flags.keys.size(); ++i)
        m.flags.emplace_back(flags.keys[i], d.boolean(flags.items[i], R + ".flags." + flags.keys[i]));
    m.model_id = d.req_str(root, "modelID", R);
    if (const JVal* h = Decoder::opt(root, "sourceSnapshotHash")) d.str(*h, R + ".sourceSnapshotHash");
    if (const JVal* b = Decoder::opt(root, "bitWidthOverridesHonored"))
        d.integer(*b, R + ".bitWidthOverridesHonored");

    const std::string A = "manifest.arch";
    const JVal& a = d.object(d.req(root, "arch", R), A);
    m.hidden = d.req_int(a, "hiddenSize", A);
    m.ffn = d.req_int(a, "ffnIntermediate", A);
    m.moe_inter = d.req_int(a, "moeIntermediateSize", A);
    m.heads = d.req_int(a, "numHeads", A);
    m.kv_heads = d.req_int(a, "numKVHeads", A);
    m.full_kv_heads = d.req_int(a, "numFullKVHeads", A);
    m.head_dim = d.req_int(a, "headDim", A);
    m.full_head_dim = d.req_int(a, "fullHeadDim", A);
    m.vocab = d.req_int(a, "vocabSize", A);
    m.sliding_window = d.req_int(a, "slidingWindow", A);
    m.softcap = d.req_real(a, "finalLogitSoftcap", A);
    m.rope = d.req_real(a, "ropeTheta", A);
    m.full_rope = d.req_real(a, "fullRopeTheta", A);
    m.partial_rotary = d.req_real(a, "partialRotaryFactor", A);
    m.arch_layers = d.req_int(a, "numLayers", A);
    m.arch_experts = d.req_int(a, "numExperts", A);
    m.top_k = d.req_int(a, "topKExperts", A);
    d.req_bool(a, "tieWordEmbeddings", A);
    d.req_bool(a, "attentionKEqV", A);
    m.activation = d.req_str(a, "hiddenActivation", A);
    const JVal& mask = d.array(d.req(a, "fullAttentionLayerMask", A), A + ".fullAttentionLayerMask");
    for (const JVal& e : mask.items) m.full_mask.push_back(d.integer(e, A + ".fullAttentionLayerMask[]"));
    if (const JVal* f = Decoder::opt(a, "family")) {
        m.has_family = true;
        m.family = d.str(*f, A + ".family");
    }
    if (const JVal* k = Decoder::opt(a, "layerKinds")) {
        m.has_kinds = true;
        for (const JVal& e : d.array(*k, A + ".layerKinds").items)
            m.kinds.push_back(d.str(e, A + ".layerKinds[]"));
    }
    if (const JVal* l = Decoder::opt(a, "linearAttention")) {
        const std::string L = A + ".linearAttention";
        d.object(*l, L);
        m.has_linear = true;
        m.lin_key_heads = d.req_int(*l, "numKeyHeads", L);
        m.lin_value_heads = d.req_int(*l, "numValueHeads", L);
        m.lin_key_dim = d.req_int(*l, "keyHeadDim", L);
        m.lin_value_dim = d.req_int(*l, "valueHeadDim", L);
        m.lin_conv = d.req_int(*l, "convKernelDim", L);
        m.lin_layers = d.req_int(*l, "layerCount", L);
    }

    if (const JVal* q = Decoder::opt(root, "quant")) {
        d.object(*q, "manifest.quant");
        m.has_quant = true;
        m.embedding = decode_slot(d, *q, "embedding");
        m.attention = decode_slot(d, *q, "attention");
        m.router = decode_slot(d, *q, "router");
        m.shared_expert = decode_slot(d, *q, "sharedExpert");
        m.routed_expert = decode_slot(d, *q, "routedExpert");
    }
    if (const JVal* v = Decoder::opt(root, "vision")) {
        d.object(*v, "manifest.vision");
        m.has_vision = true;
        m.vision_path = d.req_str(*v, "weightsPath", "manifest.vision");
        m.vision_payload = d.req_u64(*v, "payloadBytes", "manifest.vision");
    }
    if (const JVal* v = Decoder::opt(root, "draft")) {
        d.object(*v, "manifest.draft");
        m.has_draft = true;
        m.draft_path = d.req_str(*v, "weightsPath", "manifest.draft");
        m.draft_payload = d.req_u64(*v, "payloadBytes", "manifest.draft");
    }

    const JVal& files = d.object(d.req(root, "files", R), R + ".files");
    for (size_t i = 0; i < files.keys.size(); ++i) {
        const std::string P = R + ".files." + files.keys[i];
        const JVal& f = d.object(files.items[i], P);
        FileEntry e;
        e.size = d.req_u64(f, "size", P);
        e.sha256 = d.req_str(f, "sha256", P);
        m.file_index[files.keys[i]] = m.files.size();
        m.files.emplace_back(files.keys[i], std::move(e));
    }
    m.experts_per_layer = d.req_int(root, "expertsPerLayer", R);
    m.num_layers = d.req_int(root, "numLayers", R);
    m.expert_stride = d.req_u64(root, "expertStride", R);
    return m;
}

bool is_known_flag(const std::string& f) {
    static const char* const known[] = {"streamingPresent", "turboQuantKV", "aneSharedExpert",
                                        "visionTower", "mtpDraft", "linearAttention"};
    for (const char* k : known)
        if (f == k) return true;
    return false;
}

// MoEPackManifestCodec.validateLinearAttentionSection (MoEPackManifestV1.swift:497-559).
void validate_linear_attention(const Manifest& m) {
    if (m.has_family && m.family.empty()) corrupt("manifest.arch.family: empty family name");
    if (m.has_kinds) {
        if ((int64_t)m.kinds.size() != m.arch_layers)
            corrupt("manifest.arch.layerKinds: expected " + std::to_string(m.arch_layers) +
                    " entries, got " + std::to_string(m.kinds.size()));
        for (const auto& k : m.kinds)
            if (k != "full_attention" && k != "sliding_attention" && k != "linear_attention")
                corrupt("manifest.arch.layerKinds: unknown v1 layer kind");
        bool agree = m.kinds.size() == m.full_mask.size();
        for (size_t i = 0; agree && i < m.kinds.size(); ++i)
            agree = m.full_mask[i] == (m.kinds[i] == "full_attention" ? 1 : 0);
        if (!agree) corrupt("manifest.arch.layerKinds: disagrees with fullAttentionLayerMask");
    }
    const bool flagged = m.flag("linearAttention");
    if (!m.has_linear) {
        if (flagged)
            corrupt("manifest.arch.linearAttention: flags.linearAttention is set but the section "
                    "is absent");
        return;
    }
    if (!flagged)
        corrupt("manifest.flags.linearAttention: linearAttention section present but the flag "
                "is not set");
    if (m.version_minor < kVersionMinorLinearAttention)
        corrupt("manifest.version: linear attention requires minor >= 3");
    if (!m.has_kinds)
        corrupt("manifest.arch.layerKinds: a linear-attention model must say which layers are "
                "which");
    if (!(m.lin_key_heads > 0 && m.lin_value_heads > 0 && m.lin_key_dim > 0 &&
          m.lin_value_dim > 0 && m.lin_conv > 0 && m.lin_layers > 0 &&
          m.lin_layers <= m.arch_layers))
        corrupt("manifest.arch.linearAttention: invalid linear-attention values");
    const int64_t counted = std::count(m.kinds.begin(), m.kinds.end(), "linear_attention");
    if (counted != m.lin_layers)
        corrupt("manifest.arch.linearAttention.layerCount: layerKinds has " +
                std::to_string(counted) + " linear layers, section says " +
                std::to_string(m.lin_layers));
}

// The flag/section pairing, minor version and file checks of the vision and
// drafter sections (MoEPackManifestV1.swift:565-625, 630-650). Their geometry
// is not restated: this reader loads no tower or drafter weights.
void validate_optional_section(const Manifest& m, bool present, const char* flag_name,
                               const char* section, int min_minor, const std::string& path,
                               uint64_t payload) {
    const bool flagged = m.flag(flag_name);
    const std::string S = std::string("manifest.") + section;
    if (!present) {
        if (flagged)
            corrupt(S + ": flags." + flag_name + " is set but the " + section +
                    " section is absent");
        return;
    }
    if (!flagged)
        corrupt(std::string("manifest.flags.") + flag_name + ": " + section +
                " section present but the flag is not set");
    if (m.version_minor < min_minor)
        corrupt("manifest.version: " + std::string(section) + " requires minor >= " +
                std::to_string(min_minor));
    validate_relative_path(path, S + ".weightsPath");
    const FileEntry* e = m.file(path);
    if (!e) corrupt(S + ".weightsPath: " + path + " is not declared in manifest.files");
    if (!(e->size > payload))
        corrupt(S + ".payloadBytes: payload " + std::to_string(payload) + " does not fit in " +
                std::to_string(e->size) + " bytes");
}

// MoEPackManifestCodec.validate (MoEPackManifestV1.swift:378-478).
void codec_validate(const Manifest& m) {
    if (m.model_id.empty() || m.num_layers <= 0 || m.experts_per_layer <= 0 ||
        m.expert_stride == 0 || m.expert_stride % kAlignmentBytes)
        corrupt("manifest: invalid dimensions or stride");
    if (m.arch_layers != m.num_layers || m.arch_experts != m.experts_per_layer)
        corrupt("manifest.arch: dimensions disagree with streaming metadata");
    const bool arch_ok =
        m.hidden > 0 && m.ffn > 0 && m.moe_inter > 0 && m.heads > 0 && m.kv_heads > 0 &&
        m.full_kv_heads > 0 && m.head_dim > 0 && m.full_head_dim > 0 && m.vocab > 0 &&
        (m.sliding_window > 0 || m.has_linear) && m.sliding_window >= 0 && m.top_k > 0 &&
        m.top_k <= m.arch_experts && std::isfinite(m.softcap) && std::isfinite(m.rope) &&
        m.rope > 0 && std::isfinite(m.full_rope) && m.full_rope > 0 &&
        std::isfinite(m.partial_rotary) && m.partial_rotary >= 0 && m.partial_rotary <= 1 &&
        !m.activation.empty() && (int64_t)m.full_mask.size() == m.arch_layers &&
        std::all_of(m.full_mask.begin(), m.full_mask.end(),
                    [](int64_t v) { return v == 0 || v == 1; });
    if (!arch_ok) corrupt("manifest.arch: invalid architecture values");
    if (m.has_quant) {
        const std::pair<const char*, const QuantSlot*> slots[] = {
            {"embedding", &m.embedding},   {"attention", &m.attention},
            {"router", &m.router},         {"sharedExpert", &m.shared_expert},
            {"routedExpert", &m.routed_expert}};
        for (const auto& s : slots) {
            const QuantSlot& q = *s.second;
            if (!(q.weight_bits > 0 && q.weight_bits <= 32 && q.group_size > 0 &&
                  !q.scheme.empty() && !q.scale_type.empty() && !q.bias_type.empty()))
                corrupt(std::string("manifest.quant.") + s.first + ": invalid quantization values");
        }
    }
    validate_linear_attention(m);
    validate_optional_section(m, m.has_vision, "visionTower", "vision", kVersionMinorVision,
                              m.vision_path, m.vision_payload);
    validate_optional_section(m, m.has_draft, "mtpDraft", "draft", kVersionMinorDraft,
                              m.draft_path, m.draft_payload);

    // Paths in sorted order, as the reference walks them.
    std::vector<std::string> paths;
    for (const auto& f : m.files) paths.push_back(f.first);
    std::sort(paths.begin(), paths.end());
    std::unordered_map<std::string, std::string> canonical;
    for (const auto& path : paths) {
        const std::string field = "manifest.files." + path;
        validate_relative_path(path, field);
        const std::string key = filesystem_key(path);
        if (!canonical.emplace(key, path).second)
            corrupt(field + ": filesystem-equivalent duplicate path");
        static const char* const reserved[] = {"manifest.json", "verified-install.json"};
        bool is_reserved = key == "tokenizer";
        for (const char* r : reserved)
            if (key == r || key.rfind(std::string(r) + "/", 0) == 0) is_reserved = true;
        if (is_reserved) corrupt(field + ": reserved artifact filename");
        const std::string& sha = m.file(path)->sha256;
        const bool hex = sha.size() == 64 &&
                         std::all_of(sha.begin(), sha.end(), [](char c) {
                             return (c >= '0' && c <= '9') || (c >= 'a' && c <= 'f') ||
                                    (c >= 'A' && c <= 'F');
                         });
        if (!hex) corrupt(field + ".sha256: expected 64 hexadecimal characters");
    }
    for (const auto& kv : canonical) {
        std::string key = kv.first;
        for (size_t slash = key.rfind('/'); slash != std::string::npos && slash > 0;
             slash = key.rfind('/')) {
            key.resize(slash);
            if (canonical.count(key))
                corrupt("manifest.files." + kv.second +
                        ": file path collides with a directory prefix");
        }
    }
}

// ManifestReader.validateQuant (ManifestReader.swift:250-313).
struct QuantSummary {
    uint32_t group_size = 0;
    bool symmetric = false;
};

QuantSummary validate_quant(const Manifest& m) {
    const bool gemma4 = !m.has_family;
    struct Slot {
        const char* name;
        const QuantSlot* q;
        std::vector<int64_t> allowed;
    };
    const std::vector<int64_t> wide = gemma4 ? std::vector<int64_t>{4} : std::vector<int64_t>{4, 8};
    const Slot slots[] = {{"embedding", &m.embedding, wide},
                          {"attention", &m.attention, wide},
                          {"router", &m.router, {8, 16}},
                          {"sharedExpert", &m.shared_expert, {4, 8}},
                          {"routedExpert", &m.routed_expert, {4}}};
    for (const Slot& s : slots) {
        const QuantSlot& q = *s.q;
        const std::string unsupported = std::string("unsupported quantization for ") + s.name;
        if (std::find(s.allowed.begin(), s.allowed.end(), q.weight_bits) == s.allowed.end())
            corrupt(unsupported);
        const std::string scheme = lower_ascii(q.scheme), st = lower_ascii(q.scale_type),
                          bt = lower_ascii(q.bias_type);
        if (q.weight_bits == 16) {
            if (!(scheme == "bf16" && st == "none" && bt == "none")) corrupt(unsupported);
        } else if (scheme == "sym") {
            if (!(q.weight_bits == 4 && st == "bf16" && bt == "none")) corrupt(unsupported);
        } else {
            if (!(scheme == "affine" && st == "bf16" && bt == "bf16")) corrupt(unsupported);
        }
    }
    int first_sym = -1;
    std::string listing;
    bool disagree = false;
    for (const Slot& s : slots) {
        if (s.q->weight_bits != 4) continue;
        const int sym = lower_ascii(s.q->scheme) == "sym";
        if (first_sym < 0) first_sym = sym;
        else if (sym != first_sym) disagree = true;
        listing += (listing.empty() ? "" : ", ") + std::string(s.name) + "=" + s.q->scheme;
    }
    if (disagree) corrupt("4-bit slots disagree on the affine scheme: " + listing);
    const int64_t group = m.embedding.group_size;
    if (group != 32 && group != 64)
        corrupt("unsupported affine group size " + std::to_string(group));
    for (const Slot& s : slots)
        if (s.q->group_size != group)
            corrupt(std::string(s.name) + " group size " + std::to_string(s.q->group_size) +
                    " disagrees with the model's " + std::to_string(group));
    return QuantSummary{(uint32_t)group, first_sym == 1};
}

// ManifestReader.decode + validate (ManifestReader.swift:182-245), less the
// field-by-field comparison with a compiled ArchConfig (the caller compares
// the dimensions reported by tsg_moepack_get_info).
Manifest read_manifest(const char* data, size_t n, QuantSummary* quant) {
    JVal root;
    JsonReader(data, n, "manifest.json").parse(root);
    Manifest m = decode_manifest(root);
    if (m.magic != "MOEPACK" && m.magic != "GTURBO")
        throw_error(TSG_ERR_FORMAT, "notAMoEPackDirectory: manifest.magic is \"" + m.magic + "\"");
    if (m.version_major != kVersionMajor || m.version_minor < 0)
        throw_error(TSG_ERR_FORMAT, "unsupportedVersion: major " + std::to_string(m.version_major) +
                                        ", minor " + std::to_string(m.version_minor));
    for (const auto& f : m.flags)
        if (!is_known_flag(f.first)) throw_error(TSG_ERR_FORMAT, "unknownFlag: " + f.first);
    if (m.expert_stride % kAlignmentBytes)
        throw_error(TSG_ERR_FORMAT, "expertStrideNotPageAligned: stride " +
                                        std::to_string(m.expert_stride) + ", page size 16384");
    codec_validate(m);
    if (m.flag("turboQuantKV")) corrupt("manifest requests removed TurboQuant KV runtime support");
    if (m.has_vision && !m.file(m.vision_path))
        throw_error(TSG_ERR_FORMAT, "missingFile: " + m.vision_path);
    if (m.has_draft && !m.file(m.draft_path))
        throw_error(TSG_ERR_FORMAT, "missingFile: " + m.draft_path);
    *quant = m.has_quant ? validate_quant(m) : QuantSummary{};
    for (const char* f : {"model_weights.bin", "packed_experts/layout.json"})
        if (!m.file(f)) throw_error(TSG_ERR_FORMAT, std::string("missingFile: ") + f);
    return m;
}

// --------------------------------------------------------------- layout ----

struct SubTensor {
    std::string name;
    uint64_t offset = 0, size = 0;
    uint32_t dtype = 0;  // MoEPackFormatV1.DType: 0 U32, 1 BF16
    std::vector<uint32_t> shape;
    int64_t bits = 0;    // 0: not given
};

struct Expert {
    int64_t logical = 0, physical = 0;
    uint64_t offset = 0, size = 0;
    std::vector<SubTensor> tensors;
    const SubTensor* tensor(const std::string& name) const {
        for (const auto& t : tensors)
            if (t.name == name) return &t;
        return nullptr;
    }
};

struct Layer {
    int64_t id = 0;
    std::string file;
    std::vector<Expert> experts;  // indexed by logical expert id
};

struct Layout {
    uint64_t expert_stride = 0;
    int64_t num_layers = 0, experts_per_layer = 0;
    std::vector<Layer> layers;    // indexed by layer id
};

uint64_t checked_mul(uint64_t a, uint64_t b, const char* field) {
    uint64_t r;
    if (__builtin_mul_overflow(a, b, &r)) corrupt(std::string(field) + ": arithmetic overflow");
    return r;
}
uint64_t checked_add(uint64_t a, uint64_t b, const std::string& field) {
    uint64_t r;
    if (__builtin_add_overflow(a, b, &r)) corrupt(field + ": arithmetic overflow");
    return r;
}

// Decode (MoEPackPackedExpertsLayoutV1.swift:49-68), structural validation
// (:84-176) and the runtime reader's ordering (PackedExpertsLayout.swift:
// 98-114: layers by id, experts by logical id).
Layout read_layout(const char* data, size_t n) {
    JVal root;
    JsonReader(data, n, "packed_experts/layout.json").parse(root);
    Decoder d{"packed_experts/layout.json"};
    const std::string R = "layout";
    d.object(root, R);
    Layout out;
    out.expert_stride = d.req_u64(root, "expertStride", R);
    out.num_layers = d.req_int(root, "numLayers", R);
    out.experts_per_layer = d.req_int(root, "expertsPerLayer", R);
    const JVal& layers = d.array(d.req(root, "layers", R), R + ".layers");

    // Decode every layer before validating, as Codable does.
    std::vector<Layer> wire;
    std::vector<std::vector<std::pair<bool, bool>>> explicit_ids;  // (expert given, rank given)
    for (size_t li = 0; li < layers.items.size(); ++li) {
        const std::string L = R + ".layers[" + std::to_string(li) + "]";
        const JVal& lj = d.object(layers.items[li], L);
        Layer layer;
        layer.id = d.req_int(lj, "layer", L);
        layer.file = d.req_str(lj, "file", L);
        const JVal& ex = d.array(d.req(lj, "experts", L), L + ".experts");
        std::vector<std::pair<bool, bool>> given;
        for (size_t ei = 0; ei < ex.items.size(); ++ei) {
            const std::string E = L + ".experts[" + std::to_string(ei) + "]";
            const JVal& ej = d.object(ex.items[ei], E);
            Expert e;
            const JVal* lid = Decoder::opt(ej, "expert");
            const JVal* prk = Decoder::opt(ej, "physicalRank");
            e.logical = lid ? d.integer(*lid, E + ".expert") : (int64_t)ei;
            e.physical = prk ? d.integer(*prk, E + ".physicalRank") : e.logical;
            given.emplace_back(lid != nullptr, prk != nullptr);
            e.offset = d.req_u64(ej, "offset", E);
            e.size = d.req_u64(ej, "size", E);
            const JVal& ts = d.object(d.req(ej, "tensors", E), E + ".tensors");
            for (size_t ti = 0; ti < ts.keys.size(); ++ti) {
                const std::string T = E + ".tensors." + ts.keys[ti];
                const JVal& tj = d.object(ts.items[ti], T);
                SubTensor t;
                t.name = ts.keys[ti];
                t.offset = d.req_u64(tj, "offset", T);
                t.size = d.req_u64(tj, "size", T);
                const std::string dtype = d.req_str(tj, "dtype", T);
                t.dtype = dtype == "U32" ? 0u : dtype == "BF16" ? 1u : 0xFFu;
                for (const JVal& s : d.array(d.req(tj, "shape", T), T + ".shape").items) {
                    const uint64_t v = d.unsigned64(s, T + ".shape[]");
                    if (v > UINT32_MAX) d.bad(T + ".shape[]", "value does not fit UInt32");
                    t.shape.push_back((uint32_t)v);
                }
                if (const JVal* b = Decoder::opt(tj, "bits")) {
                    t.bits = d.integer(*b, T + ".bits");
                    if (t.bits == 0) t.bits = -1;  // present but zero: invalid below
                }
                e.tensors.push_back(std::move(t));
            }
            layer.experts.push_back(std::move(e));
        }
        wire.push_back(std::move(layer));
        explicit_ids.push_back(std::move(given));
    }

    if (!(out.num_layers > 0 && out.experts_per_layer > 0 && out.expert_stride > 0 &&
          out.expert_stride % kAlignmentBytes == 0 && (int64_t)wire.size() == out.num_layers))
        corrupt("layout: invalid dimensions or stride");
    std::unordered_set<int64_t> layer_ids;
    std::unordered_set<std::string> layer_files;
    for (size_t li = 0; li < wire.size(); ++li) {
        const Layer& layer = wire[li];
        if (!(layer.id >= 0 && layer.id < out.num_layers && layer_ids.insert(layer.id).second))
            corrupt("layout.layers: duplicate or invalid layer");
        const std::string F = "layout.layers[" + std::to_string(layer.id) + "]";
        validate_basename(layer.file, F + ".file");
        const std::string key = filesystem_key(layer.file);
        if (key == "layout.json") corrupt(F + ".file: reserved packed-expert filename");
        if (!layer_files.insert(key).second) corrupt(F + ".file: duplicate layer filename");
        if ((int64_t)layer.experts.size() != out.experts_per_layer)
            corrupt(F + ".experts: wrong expert count");
        const auto& given = explicit_ids[li];
        const bool all_explicit = std::all_of(given.begin(), given.end(),
                                              [](const auto& g) { return g.first; });
        const bool all_positional = std::none_of(given.begin(), given.end(),
                                                 [](const auto& g) { return g.first; });
        if (!(all_explicit || all_positional))
            corrupt(F + ".experts: expert ids must be either all explicit or all positional");
        std::unordered_set<int64_t> logical_ids, ranks;
        std::unordered_set<uint64_t> offsets;
        for (const Expert& e : layer.experts) {
            if (!(e.logical >= 0 && e.logical < out.experts_per_layer && e.physical >= 0 &&
                  e.physical < out.experts_per_layer && logical_ids.insert(e.logical).second &&
                  ranks.insert(e.physical).second && offsets.insert(e.offset).second))
                corrupt(F + ".experts: duplicate or invalid expert mapping");
            const std::string X = "expert[" + std::to_string(e.logical) + "]";
            const uint64_t expected = checked_mul((uint64_t)e.physical, out.expert_stride,
                                                  "expert.offset");
            if (e.offset != expected || e.size != out.expert_stride)
                corrupt(X + ": offset or size does not match physical rank");
            std::vector<std::pair<std::pair<uint64_t, uint64_t>, const std::string*>> ranges;
            for (const SubTensor& t : e.tensors) {
                const bool ok = t.dtype != 0xFFu && !t.name.empty() && t.size > 0 &&
                                !t.shape.empty() &&
                                std::all_of(t.shape.begin(), t.shape.end(),
                                            [](uint32_t v) { return v > 0; }) &&
                                (t.bits == 0 || (t.bits > 0 && t.bits <= 32));
                if (!ok) corrupt(X + ".tensors." + t.name + ": invalid dtype or shape");
                const uint64_t end = checked_add(t.offset, t.size, "tensor." + t.name + ".range");
                if (end > e.size) corrupt(X + ".tensors." + t.name + ": range exceeds expert blob");
                ranges.push_back({{t.offset, end}, &t.name});
            }
            std::sort(ranges.begin(), ranges.end(),
                      [](const auto& a, const auto& b) { return a.first < b.first; });
            for (size_t i = 1; i < ranges.size(); ++i)
                if (ranges[i - 1].first.second > ranges[i].first.first)
                    corrupt(X + ".tensors: overlapping ranges " + *ranges[i - 1].second + " and " +
                            *ranges[i].second);
        }
    }

    out.layers.resize(out.num_layers);
    for (Layer& layer : wire) {
        std::vector<Expert> by_logical(layer.experts.size());
        for (Expert& e : layer.experts) by_logical[e.logical] = std::move(e);
        layer.experts = std::move(by_logical);
        const int64_t id = layer.id;
        out.layers[id] = std::move(layer);
    }
    return out;
}

// MoEPackV1StructuralValidator.crossValidate (MoEPackPackedExpertsLayoutV1.swift:186-211).
void cross_validate(const Manifest& m, const Layout& l) {
    if (m.num_layers != l.num_layers || m.experts_per_layer != l.experts_per_layer ||
        m.expert_stride != l.expert_stride)
        corrupt("layout.json: manifest/layout: dimension mismatch");
    const uint64_t layer_size = checked_mul((uint64_t)l.experts_per_layer, l.expert_stride,
                                            "layout.layerSize");
    for (const Layer& layer : l.layers) {
        const std::string path = "packed_experts/" + layer.file;
        const FileEntry* f = m.file(path);
        if (!f || f->size != layer_size)
            corrupt("layout.json: manifest.files." + path + ": missing or wrong layer size");
    }
}

// ------------------------------------------------------------ directory ----

// MoEPackModelDirectory.openFile: each component opened with O_NOFOLLOW under
// the root, the last one O_NONBLOCK (a FIFO cannot stall the reader) and
// required to be a regular file.
int open_in_directory(int root_fd, const std::string& rel) {
    try {
        validate_relative_path(rel, "path." + rel);
    } catch (const LoadError& e) {
        corrupt("unsafe path " + rel + ": " + e.message);
    }
    int dir = fcntl(root_fd, F_DUPFD_CLOEXEC, 0);
    if (dir < 0) throw_error(TSG_ERR_IO, "posixFailed: fcntl(F_DUPFD_CLOEXEC, model root): " +
                                             std::string(strerror(errno)));
    size_t start = 0;
    for (;;) {
        const size_t slash = rel.find('/', start);
        const std::string comp = rel.substr(start, slash == std::string::npos ? std::string::npos
                                                                           : slash - start);
        const bool last = slash == std::string::npos;
        const int flags = last ? (O_RDONLY | O_NONBLOCK | O_NOFOLLOW | O_CLOEXEC)
                               : (O_RDONLY | O_DIRECTORY | O_NOFOLLOW | O_CLOEXEC);
        const int next = openat(dir, comp.c_str(), flags);
        const int saved = errno;
        close(dir);
        if (next < 0) {
            if (saved == ENOENT) throw_error(TSG_ERR_IO, "missingFile: " + rel);
            throw_error(TSG_ERR_IO, "posixFailed: openat(" + rel + "): " + strerror(saved));
        }
        if (last) {
            struct stat st;
            if (fstat(next, &st) != 0 || !S_ISREG(st.st_mode)) {
                close(next);
                throw_error(TSG_ERR_IO, "posixFailed: fstat(" + rel + "): not a regular file");
            }
            return next;
        }
        dir = next;
        start = slash + 1;
    }
}

void pread_all(int fd, void* buf, uint64_t n, uint64_t off, const std::string& rel) {
    uint64_t done = 0;
    while (done < n) {
        const ssize_t got = pread(fd, static_cast<char*>(buf) + done, n - done, (off_t)(off + done));
        if (got < 0 && errno == EINTR) continue;
        if (got <= 0)
            throw_error(TSG_ERR_IO, "posixFailed: pread(" + rel + "): " +
                                        (got < 0 ? strerror(errno) : "unexpected end of file"));
        done += (uint64_t)got;
    }
}

uint64_t file_size(int fd, const std::string& rel) {
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 0)
        throw_error(TSG_ERR_IO, "posixFailed: fstat(" + rel + ")");
    return (uint64_t)st.st_size;
}

// readMetadata: the size cap is checked before any byte is read.
std::string read_metadata(int root_fd, const std::string& rel, uint64_t max_bytes) {
    const int fd = open_in_directory(root_fd, rel);
    std::string data;
    try {
        const uint64_t size = file_size(fd, rel);
        if (size > max_bytes)
            corrupt(rel + " size " + std::to_string(size) + " exceeds metadata cap " +
                    std::to_string(max_bytes));
        data.resize(size);
        if (size) pread_all(fd, &data[0], size, 0, rel);
    } catch (...) {
        close(fd);
        throw;
    }
    close(fd);
    return data;
}

struct Fd {
    int fd = -1;
    ~Fd() { if (fd >= 0) close(fd); }
};

}  // namespace

// ------------------------------------------------------------------ ABI ----

struct tsg_moepack {
    Manifest manifest;
    QuantSummary quant;
    bool has_layout = false;
    Layout layout;
    int root_fd = -1;  // open directory of an installed pack, -1 when parsed from memory
    ~tsg_moepack() { if (root_fd >= 0) close(root_fd); }
};

namespace {

template <class F>
tsg_status guarded(F&& body) {
    try {
        return body();
    } catch (const LoadError& e) {
        return tsg::fail(e.status, "%s", e.message.c_str());
    } catch (const std::bad_alloc&) {
        return tsg::fail(TSG_ERR_FORMAT, "indexCorrupt: out of host memory while parsing");
    }
}

void build_pack(tsg_moepack* pack, const char* manifest, size_t manifest_len,
                const char* layout, size_t layout_len, bool with_layout) {
    pack->manifest = read_manifest(manifest, manifest_len, &pack->quant);
    if (with_layout) {
        pack->layout = read_layout(layout, layout_len);
        cross_validate(pack->manifest, pack->layout);
        pack->has_layout = true;
    }
}

const Layer& layer_of(const tsg_moepack* pack, uint32_t layer) {
    if (!pack->has_layout)
        throw_error(TSG_ERR_INVALID_ARGUMENT, "the pack was opened without packed_experts/layout.json");
    if ((int64_t)layer >= pack->layout.num_layers)
        throw_error(TSG_ERR_INVALID_ARGUMENT,
                    "layer " + std::to_string(layer) + " not in 0..<" +
                        std::to_string(pack->layout.num_layers));
    return pack->layout.layers[layer];
}

// routedExpertOffsets (ModelExpertIO.swift:56-84): offsets of expert 0's
// sub-tensors; a blob without `<role>_biases` aliases the bias to the scales.
tsg_expert_offsets routed_offsets(const Layer& layer) {
    const Expert& e = layer.experts[0];
    auto off = [&](const std::string& role) -> uint32_t {
        const SubTensor* t = e.tensor(role);
        if (!t || t->offset > UINT32_MAX)
            corrupt("invalid routed expert metadata for role " + role);
        return (uint32_t)t->offset;
    };
    auto bias = [&](const std::string& role) -> uint32_t {
        return e.tensor(role + "_biases") ? off(role + "_biases") : off(role + "_scales");
    };
    tsg_expert_offsets o;
    o.gate_w = off("gate");
    o.gate_s = off("gate_scales");
    o.gate_b = bias("gate");
    o.up_w = off("up");
    o.up_s = off("up_scales");
    o.up_b = bias("up");
    o.down_w = off("down");
    o.down_s = off("down_scales");
    o.down_b = bias("down");
    return o;
}

}  // namespace

extern "C" tsg_status tsg_moepack_parse(const char* manifest_json, uint64_t manifest_len,
                                        const char* layout_json, uint64_t layout_len,
                                        tsg_moepack** out) {
    if (!out || (!manifest_json && manifest_len))
        return tsg::fail(TSG_ERR_INVALID_ARGUMENT, "NULL manifest/out");
    *out = nullptr;
    if (!layout_json && layout_len) return tsg::fail(TSG_ERR_INVALID_ARGUMENT, "NULL layout");
    return guarded([&] {
        auto* pack = new tsg_moepack();
        try {
            build_pack(pack, manifest_json ? manifest_json : "", manifest_len, layout_json,
                       layout_len, layout_json != nullptr);
        } catch (...) {
            delete pack;
            throw;
        }
        *out = pack;
        return TSG_OK;
    });
}

extern "C" tsg_status tsg_moepack_open(const char* directory, uint64_t manifest_max_bytes,
                                       uint64_t layout_max_bytes, tsg_moepack** out) {
    if (!directory || !out) return tsg::fail(TSG_ERR_INVALID_ARGUMENT, "NULL directory/out");
    *out = nullptr;
    return guarded([&] {
        const int root = open(directory, O_RDONLY | O_DIRECTORY | O_CLOEXEC);
        if (root < 0)
            throw_error(TSG_ERR_IO, std::string("posixFailed: open(") + directory + "): " +
                                        strerror(errno));
        auto* pack = new tsg_moepack();
        pack->root_fd = root;
        try {
            std::string manifest;
            try {
                manifest = read_metadata(root, "manifest.json",
                                         manifest_max_bytes ? manifest_max_bytes : kManifestMaxBytes);
            } catch (const LoadError& e) {
                if (e.message.rfind("missingFile", 0) == 0)
                    throw_error(TSG_ERR_IO, std::string("partialInstall: ") + directory);
                throw;
            }
            pack->manifest = read_manifest(manifest.data(), manifest.size(), &pack->quant);
            const std::string layout = read_metadata(
                root, "packed_experts/layout.json", layout_max_bytes ? layout_max_bytes : kLayoutMaxBytes);
            pack->layout = read_layout(layout.data(), layout.size());
            cross_validate(pack->manifest, pack->layout);
            pack->has_layout = true;
        } catch (...) {
            delete pack;
            throw;
        }
        *out = pack;
        return TSG_OK;
    });
}

extern "C" void tsg_moepack_close(tsg_moepack* pack) { delete pack; }

extern "C" tsg_status tsg_moepack_get_info(const tsg_moepack* pack, tsg_moepack_info* out) {
    if (!pack || !out) return tsg::fail(TSG_ERR_INVALID_ARGUMENT, "NULL pack/out");
    const Manifest& m = pack->manifest;
    tsg_moepack_info info;
    memset(&info, 0, sizeof info);
    info.num_layers = (uint32_t)m.num_layers;
    info.experts_per_layer = (uint32_t)m.experts_per_layer;
    info.expert_stride = m.expert_stride;
    info.hidden_size = (uint32_t)m.hidden;
    info.moe_intermediate_size = (uint32_t)m.moe_inter;
    info.top_k = (uint32_t)m.top_k;
    info.version_minor = (uint32_t)m.version_minor;
    info.legacy_magic = m.magic == "GTURBO";
    info.has_quant = m.has_quant;
    info.affine_group_size = pack->quant.group_size;
    info.symmetric = pack->quant.symmetric;
    info.routed_weight_bits = m.has_quant ? (uint32_t)m.routed_expert.weight_bits : 0;
    info.shared_weight_bits = m.has_quant ? (uint32_t)m.shared_expert.weight_bits : 0;
    info.router_weight_bits = m.has_quant ? (uint32_t)m.router.weight_bits : 0;
    info.has_layout = pack->has_layout;
    info.is_gemma4 = !m.has_family;
    snprintf(info.family, sizeof info.family, "%s", m.family.c_str());
    *out = info;
    return TSG_OK;
}

extern "C" tsg_status tsg_moepack_routed_offsets(const tsg_moepack* pack, uint32_t layer,
                                                 tsg_expert_offsets* out) {
    if (!pack || !out) return tsg::fail(TSG_ERR_INVALID_ARGUMENT, "NULL pack/out");
    return guarded([&] {
        *out = routed_offsets(layer_of(pack, layer));
        return TSG_OK;
    });
}

extern "C" tsg_status tsg_moepack_physical_offsets(const tsg_moepack* pack, uint32_t layer,
                                                   uint64_t* offsets, uint32_t count) {
    if (!pack || !offsets) return tsg::fail(TSG_ERR_INVALID_ARGUMENT, "NULL pack/offsets");
    return guarded([&] {
        const Layer& l = layer_of(pack, layer);
        if (count != l.experts.size())
            throw_error(TSG_ERR_INVALID_ARGUMENT, "count " + std::to_string(count) + " != " +
                                                      std::to_string(l.experts.size()) + " experts");
        for (size_t e = 0; e < l.experts.size(); ++e) offsets[e] = l.experts[e].offset;
        return TSG_OK;
    });
}

extern "C" tsg_status tsg_moepack_tensor(const tsg_moepack* pack, uint32_t layer, uint32_t expert,
                                         const char* name, tsg_moepack_subtensor* out) {
    if (!pack || !name || !out) return tsg::fail(TSG_ERR_INVALID_ARGUMENT, "NULL argument");
    return guarded([&] {
        const Layer& l = layer_of(pack, layer);
        if (expert >= l.experts.size())
            throw_error(TSG_ERR_INVALID_ARGUMENT, "expert " + std::to_string(expert) + " not in 0..<" +
                                                      std::to_string(l.experts.size()));
        const SubTensor* t = l.experts[expert].tensor(name);
        if (!t) throw_error(TSG_ERR_INVALID_ARGUMENT, std::string("no sub-tensor \"") + name + "\"");
        tsg_moepack_subtensor r;
        memset(&r, 0, sizeof r);
        r.offset = t->offset;
        r.size = t->size;
        r.dtype = t->dtype;
        r.bits = t->bits > 0 ? (uint32_t)t->bits : 0;
        r.rank = (uint32_t)t->shape.size();
        for (size_t i = 0; i < t->shape.size() && i < 8; ++i) r.shape[i] = t->shape[i];
        r.physical_rank = (uint32_t)l.experts[expert].physical;
        *out = r;
        return TSG_OK;
    });
}

// One layer file into HBM. The file is read in physical order through two
// pinned staging buffers (the read of one overlaps the copy of the other);
// each run of physically consecutive experts whose logical ids are also
// consecutive goes up in one copy to logical_id * stride.
namespace {

tsg_status upload_layer_file(const tsg_moepack* pack, tsg_stream stream, uint32_t layer,
                             tsg_layer* dst) {
    void* staging[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    bool recorded[2] = {false, false};
    const tsg_status st = guarded([&] {
        const Layer& l = layer_of(pack, layer);
        if (pack->root_fd < 0)
            throw_error(TSG_ERR_INVALID_ARGUMENT, "the pack was parsed from memory: no layer files");
        const tsg_expert_offsets offsets = routed_offsets(l);
        const uint64_t stride = pack->layout.expert_stride;
        const uint32_t n = (uint32_t)l.experts.size();
        int device = 0;
        uint32_t dst_experts = 0;
        uint64_t dst_stride = 0;
        tsg_expert_offsets dst_offsets;
        tsg::layer_geometry(dst, &device, &dst_experts, &dst_stride, &dst_offsets);
        if (dst_experts != n || dst_stride != stride ||
            memcmp(&dst_offsets, &offsets, sizeof offsets) != 0)
            throw_error(TSG_ERR_INVALID_ARGUMENT,
                        "destination layer geometry (" + std::to_string(dst_experts) + " x " +
                            std::to_string(dst_stride) +
                            ", offsets) differs from the pack's layer " + std::to_string(layer));
        const std::string rel = "packed_experts/" + l.file;
        Fd fd;
        fd.fd = open_in_directory(pack->root_fd, rel);
        const uint64_t expected = (uint64_t)n * stride;
        const uint64_t size = file_size(fd.fd, rel);
        if (size != expected)
            corrupt(rel + ": file is " + std::to_string(size) + " bytes, layout says " +
                    std::to_string(expected));
        hipError_t e = hipSetDevice(device);
        if (e != hipSuccess)
            throw_error(TSG_ERR_HIP, std::string("hipSetDevice: ") + hipGetErrorString(e));

        std::vector<uint32_t> logical_of(n);
        for (uint32_t x = 0; x < n; ++x) logical_of[l.experts[x].physical] = x;
        const uint32_t per_chunk = (uint32_t)std::max<uint64_t>(
            1, std::min<uint64_t>(n, kStagingBytes / stride));
        const uint64_t chunk_bytes = (uint64_t)per_chunk * stride;
        for (int b = 0; b < 2; ++b) {
            e = hipHostMalloc(&staging[b], chunk_bytes, hipHostMallocDefault);
            if (e != hipSuccess)
                throw_error(TSG_ERR_OUT_OF_MEMORY, std::string("pinned staging of ") +
                                                       std::to_string(chunk_bytes) +
                                                       " bytes: " + hipGetErrorString(e));
            e = hipEventCreateWithFlags(&done[b], hipEventDisableTiming);
            if (e != hipSuccess)
                throw_error(TSG_ERR_HIP, std::string("hipEventCreate: ") + hipGetErrorString(e));
        }
        const hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
        int buf = 0;
        for (uint32_t p0 = 0; p0 < n; p0 += per_chunk, buf ^= 1) {
            const uint32_t cnt = std::min(per_chunk, n - p0);
            // wait for the copy that last read this buffer
            e = recorded[buf] ? hipEventSynchronize(done[buf]) : hipSuccess;
            if (e != hipSuccess)
                throw_error(TSG_ERR_HIP, std::string("hipEventSynchronize: ") + hipGetErrorString(e));
            auto* host = static_cast<uint8_t*>(staging[buf]);
            pread_all(fd.fd, host, (uint64_t)cnt * stride, (uint64_t)p0 * stride, rel);
            for (uint32_t i = 0; i < cnt;) {
                uint32_t run = 1;
                while (i + run < cnt && logical_of[p0 + i + run] == logical_of[p0 + i] + run) ++run;
                const tsg_status s = tsg_layer_upload(dst, stream, host + (uint64_t)i * stride,
                                                      (uint64_t)run * stride,
                                                      (uint64_t)logical_of[p0 + i] * stride);
                if (s != TSG_OK) throw_error(s, tsg_last_error());
                i += run;
            }
            e = hipEventRecord(done[buf], hs);
            if (e != hipSuccess)
                throw_error(TSG_ERR_HIP, std::string("hipEventRecord: ") + hipGetErrorString(e));
            recorded[buf] = true;
        }
        for (int b = 0; b < 2; ++b) {
            e = recorded[b] ? hipEventSynchronize(done[b]) : hipSuccess;
            if (e != hipSuccess)
                throw_error(TSG_ERR_HIP, std::string("hipEventSynchronize: ") + hipGetErrorString(e));
        }
        return TSG_OK;
    });
    // On failure, drain what was queued before the staging buffers go away.
    if (st != TSG_OK && (recorded[0] || recorded[1]))
        (void)hipStreamSynchronize(reinterpret_cast<hipStream_t>(stream));
    for (int b = 0; b < 2; ++b) {
        if (done[b]) (void)hipEventDestroy(done[b]);
        if (staging[b]) (void)hipHostFree(staging[b]);
    }
    return st;
}

}  // namespace

extern "C" tsg_status tsg_moepack_upload_layer(const tsg_moepack* pack, tsg_stream stream,
                                               uint32_t layer, tsg_layer* dst) {
    if (!pack || !dst) return tsg::fail(TSG_ERR_INVALID_ARGUMENT, "NULL pack/dst");
    return upload_layer_file(pack, stream, layer, dst);
}

extern "C" tsg_status tsg_moepack_load_layer(const tsg_moepack* pack, tsg_ctx* ctx,
                                             tsg_stream stream, uint32_t layer, tsg_layer** out) {
    if (!pack || !ctx || !out) return tsg::fail(TSG_ERR_INVALID_ARGUMENT, "NULL pack/ctx/out");
    *out = nullptr;
    tsg_layer* created = nullptr;
    tsg_status st = guarded([&] {
        const Layer& l = layer_of(pack, layer);
        if (pack->root_fd < 0)
            throw_error(TSG_ERR_INVALID_ARGUMENT, "the pack was parsed from memory: no layer files");
        const tsg_expert_offsets offsets = routed_offsets(l);
        const tsg_status s = tsg_layer_create(ctx, (uint32_t)l.experts.size(),
                                              pack->layout.expert_stride, &offsets, &created);
        if (s != TSG_OK) throw_error(s, tsg_last_error());
        return TSG_OK;
    });
    if (st == TSG_OK) st = upload_layer_file(pack, stream, layer, created);
    if (st != TSG_OK) {
        if (created) tsg_layer_destroy(created);
        return st;
    }
    *out = created;
    return TSG_OK;
}
