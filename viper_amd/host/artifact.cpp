// Reader of the `.viper` v1 artifact (layout documented in
// include/viper/artifact.h; reference writer tools/convert/convert.cpp:187-284,
// reference loader include/viper/model_impl.cuh:162-257).
//
// parse() walks the sections with bounds checks and records offsets; the
// weights are never copied on the host.  upload() makes one device
// allocation for the first pass and copies each section to a 256-byte
// aligned offset in it.
#include "viper/artifact.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <climits>
#include <cstring>
#include <new>

#include <hip/hip_runtime_api.h>

namespace viper::artifact {
namespace {

constexpr u32 kVersion = 1;
constexpr usize kAlign = 256;

Status invalid(const std::string& what) { return Status(StatusCode::INVALID_ARGUMENT, "artifact: " + what); }
Status io(const std::string& what) { return Status(StatusCode::IO_ERROR, "artifact: " + what); }

// Cursor over the section stream.
struct Reader {
    const u8* data;
    usize size;
    usize pos;

    Status next(Blob* b, u64 expect, const std::string& what) {
        if (size - pos < 8) return io("truncated before the size of " + what);
        u64 n;
        std::memcpy(&n, data + pos, 8);
        pos += 8;
        if (n != expect)
            return invalid(what + ": " + std::to_string(n) + " bytes, the header implies " + std::to_string(expect));
        if (size - pos < n) return io("truncated inside " + what);
        b->offset = pos;
        b->size = n;
        pos += n;
        return Status::Ok();
    }
};

// Section sizes of a rows x cols Q4_G64 matrix.  The callers pass dimensions
// of at most INT32_MAX, so the products stay below 2^62; the checked
// multiply keeps that an invariant rather than an assumption (a wrapped size
// could match a short file and give views past its end).
bool mul_ok(u64 a, u64 b, u64* out) { return !__builtin_mul_overflow(a, b, out); }
bool q4_packed(u64 rows, u64 cols, u64* out) { return mul_ok(rows, cols / 2, out); }
bool q4_scales(u64 rows, u64 cols, u64* out) { return mul_ok(rows, (cols / 64) * 2, out); }

const char* kLinearName[N_LINEAR] = {"q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"};

usize align_up(usize v) { return (v + kAlign - 1) / kAlign * kAlign; }

}  // namespace

static Status parse_sections(const u8* data, usize size, Index* out);

// Host allocations (the index vectors, the messages) are the only thing that
// can throw in here; the API returns Status and never throws.
Status parse(const u8* data, usize size, Index* out) {
    try {
        return parse_sections(data, size, out);
    } catch (const std::bad_alloc&) {
        if (out != nullptr) *out = Index();
        return Status(StatusCode::OUT_OF_MEMORY, "artifact: host allocation failed while indexing");
    } catch (...) {
        if (out != nullptr) *out = Index();
        return Status(StatusCode::INTERNAL, "artifact: unexpected exception while indexing");
    }
}

static Status parse_sections(const u8* data, usize size, Index* out) {
    if (out == nullptr || (data == nullptr && size != 0)) return invalid("null argument");
    *out = Index();
    if (size < kHeaderBytes) return io("shorter than the 56-byte header");
    if (std::memcmp(data, "VIPER", 5) != 0) return invalid("bad magic");
    for (int i = 5; i < 16; ++i)
        if (data[i] != 0) return invalid("bad magic padding");
    u32 h[10];
    std::memcpy(h, data + 16, sizeof(h));
    Header& hd = out->header;
    hd = Header{h[0], h[1], h[2], h[3], h[4], h[5], h[6], h[7], h[8], h[9]};
    if (hd.version != kVersion) return invalid("unsupported version " + std::to_string(hd.version));
    if (hd.n_layers == 0 || hd.n_passes == 0 || hd.hidden == 0 || hd.intermediate == 0 || hd.n_heads == 0 ||
        hd.n_kv_heads == 0 || hd.head_dim == 0 || hd.vocab == 0)
        return invalid("zero dimension in the header");
    // Every dimension must fit the i32 rows/cols of a weight view (and the
    // C ABI's int shapes); products of two u32 fields cannot overflow u64.
    const u64 H = hd.hidden, I = hd.intermediate, nQ = (u64)hd.n_heads * hd.head_dim,
              nKV = (u64)hd.n_kv_heads * hd.head_dim, V = hd.vocab;
    for (const u64 dim : {H, I, nQ, nKV, V})
        if (dim > (u64)INT32_MAX) return invalid("a dimension (or n_heads*head_dim) exceeds INT32_MAX");
    if (H % 64 || I % 64 || nQ % 64) return invalid("hidden, intermediate and n_heads*head_dim must be multiples of 64");
    const u64 rows[N_LINEAR] = {nQ, nKV, nKV, H, I, I, H};
    const u64 cols[N_LINEAR] = {H, H, H, nQ, H, H, I};

    // The header's layer and pass counts are untrusted: before anything is
    // sized by them, the sections they imply must fit the file.  Per (layer,
    // pass): 7 linears of two sections each and 2 norms, each section 8 bytes
    // of size plus its data.
    u64 per_layer = 2 * (8 + H * 2);
    for (int i = 0; i < N_LINEAR; ++i) {
        u64 np = 0, ns = 0;
        if (!q4_packed(rows[i], cols[i], &np) || !q4_scales(rows[i], cols[i], &ns) ||
            __builtin_add_overflow(per_layer, 16 + np + ns, &per_layer))
            return invalid("layer size overflows");
    }
    u64 layer_passes = 0, layers_bytes = 0;
    if (!mul_ok((u64)hd.n_layers, (u64)hd.n_passes, &layer_passes) || !mul_ok(layer_passes, per_layer, &layers_bytes) ||
        layers_bytes > (u64)(size - kHeaderBytes))
        return io("the header's " + std::to_string(hd.n_layers) + " layers x " + std::to_string(hd.n_passes) +
                  " passes need more bytes than the file holds");

    Reader r{data, size, kHeaderBytes};
    out->layers.resize(hd.n_layers);
    for (u32 pass = 0; pass < hd.n_passes; ++pass) {
        for (u32 l = 0; l < hd.n_layers; ++l) {
            for (int i = 0; i < N_LINEAR; ++i) {
                const std::string name = "layer " + std::to_string(l) + " pass " + std::to_string(pass) + " " +
                                         kLinearName[i];
                LinearBlob lb;
                lb.rows = (i32)rows[i];
                lb.cols = (i32)cols[i];
                u64 np = 0, ns = 0;
                if (!q4_packed(rows[i], cols[i], &np) || !q4_scales(rows[i], cols[i], &ns))
                    return invalid(name + ": size overflows");
                Status s = r.next(&lb.packed, np, name + " packed");
                if (!s.ok()) return s;
                s = r.next(&lb.scales, ns, name + " scales");
                if (!s.ok()) return s;
                if (pass == 0) out->layers[l][i] = lb;
            }
        }
    }
    u64 ne = 0, nhp = 0, nhs = 0;
    if (!mul_ok(V, H * 2, &ne) || !q4_packed(V, H, &nhp) || !q4_scales(V, H, &nhs))
        return invalid("embedding / lm_head size overflows");
    Status s = r.next(&out->embed, ne, "embed_tokens");
    if (!s.ok()) return s;
    out->lm_head.rows = (i32)V;
    out->lm_head.cols = (i32)H;
    s = r.next(&out->lm_head.packed, nhp, "lm_head packed");
    if (!s.ok()) return s;
    s = r.next(&out->lm_head.scales, nhs, "lm_head scales");
    if (!s.ok()) return s;
    s = r.next(&out->final_norm, (u64)H * 2, "final norm");
    if (!s.ok()) return s;
    out->norms.resize(hd.n_layers);
    for (u32 pass = 0; pass < hd.n_passes; ++pass) {
        for (u32 l = 0; l < hd.n_layers; ++l) {
            std::array<Blob, 2> nb;
            const std::string name = "layer " + std::to_string(l) + " pass " + std::to_string(pass);
            s = r.next(&nb[0], (u64)H * 2, name + " input_layernorm");
            if (!s.ok()) return s;
            s = r.next(&nb[1], (u64)H * 2, name + " post_attention_layernorm");
            if (!s.ok()) return s;
            if (pass == 0) out->norms[l] = nb;
        }
    }
    if (r.pos != size) return io(std::to_string(size - r.pos) + " trailing bytes after the last section");
    return Status::Ok();
}

MappedFile::~MappedFile() {
    if (data_ != nullptr && size_ != 0) munmap(const_cast<u8*>(data_), size_);
}

Status MappedFile::open(const std::string& path) {
    if (data_ != nullptr) return invalid("file already open");
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) return io("cannot open " + path);
    struct stat st;
    if (fstat(fd, &st) != 0) {
        ::close(fd);
        return io("cannot stat " + path);
    }
    size_ = (usize)st.st_size;
    if (size_ != 0) {
        void* p = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
        if (p == MAP_FAILED) {
            ::close(fd);
            size_ = 0;
            return io("cannot map " + path);
        }
        data_ = (const u8*)p;
    }
    ::close(fd);
    return Status::Ok();
}

Status upload(const u8* data, const Index& idx, DeviceModel* out) {
    if (out == nullptr || data == nullptr) return invalid("null argument");
    *out = DeviceModel();
    // arena layout: every first-pass section at a 256-byte aligned offset
    struct Piece {
        const Blob* b;
        usize at;
    };
    std::vector<Piece> pieces;
    usize total = 0;
    auto place = [&](const Blob& b) {
        pieces.push_back({&b, total});
        total = align_up(total + (usize)b.size);
        return pieces.back().at;
    };
    std::vector<std::array<usize, 2 * N_LINEAR>> lin_at(idx.layers.size());
    for (usize l = 0; l < idx.layers.size(); ++l)
        for (int i = 0; i < N_LINEAR; ++i) {
            lin_at[l][2 * i] = place(idx.layers[l][i].packed);
            lin_at[l][2 * i + 1] = place(idx.layers[l][i].scales);
        }
    const usize embed_at = place(idx.embed);
    const usize head_p = place(idx.lm_head.packed), head_s = place(idx.lm_head.scales);
    const usize fnorm_at = place(idx.final_norm);
    std::vector<std::array<usize, 2>> norm_at(idx.norms.size());
    for (usize l = 0; l < idx.norms.size(); ++l) {
        norm_at[l][0] = place(idx.norms[l][0]);
        norm_at[l][1] = place(idx.norms[l][1]);
    }

    void* arena = nullptr;
    hipError_t e = hipMalloc(&arena, total == 0 ? kAlign : total);
    if (e != hipSuccess) return Status(e == hipErrorOutOfMemory ? StatusCode::OUT_OF_MEMORY : StatusCode::CUDA_ERROR,
                                       "artifact: device allocation of " + std::to_string(total) + " bytes");
    for (const Piece& p : pieces) {
        e = hipMemcpy((u8*)arena + p.at, data + p.b->offset, (usize)p.b->size, hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            (void)hipFree(arena);
            return Status(StatusCode::CUDA_ERROR, "artifact: copy to the device failed");
        }
    }

    auto view = [&](usize packed_at, usize scales_at, const LinearBlob& lb) {
        quant::QuantizedWeight w;
        w.qtype = quant::QType::Q4_G64;
        w.data = (u8*)arena + packed_at;
        w.scales = (u8*)arena + scales_at;
        w.rows = lb.rows;
        w.cols = lb.cols;
        w.group_size = 64;
        w.scale_enc = quant::ScaleEnc::BF16;  // the converter truncates scales to bf16
        return w;
    };
    out->arena = arena;
    out->arena_bytes = total;
    out->layers.resize(idx.layers.size());
    for (usize l = 0; l < idx.layers.size(); ++l)
        for (int i = 0; i < N_LINEAR; ++i)
            out->layers[l][i] = view(lin_at[l][2 * i], lin_at[l][2 * i + 1], idx.layers[l][i]);
    out->lm_head = view(head_p, head_s, idx.lm_head);
    out->embed = (u8*)arena + embed_at;
    out->final_norm = (u8*)arena + fnorm_at;
    out->norms.resize(idx.norms.size());
    for (usize l = 0; l < idx.norms.size(); ++l)
        out->norms[l] = {(u8*)arena + norm_at[l][0], (u8*)arena + norm_at[l][1]};
    return Status::Ok();
}

Status release(DeviceModel* model) {
    if (model == nullptr) return invalid("null argument");
    Status s = Status::Ok();
    if (model->arena != nullptr && hipFree(model->arena) != hipSuccess)
        s = Status(StatusCode::CUDA_ERROR, "artifact: device free failed");
    *model = DeviceModel();
    return s;
}

}  // namespace viper::artifact
