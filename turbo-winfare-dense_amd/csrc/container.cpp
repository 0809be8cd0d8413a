// The .g4dense container's LM-head slice loader: header parsing and validation, then the
// upload of the tied head [W|S|B] and of the final RMSNorm weight that the runner performs at
// load time (src/runner.cpp:423-443 and :488-497), straight into the device layout.
//
// The header is the reference's fixed 4096-byte little-endian record
// (include/g4dense/format.hpp:26-110, docs/G4DENSE_FORMAT.md:15-48). Only the fields this path
// reads are named below; the rest is kept as opaque bytes at its offsets.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstddef>
#include <cstdio>
#include <cstring>
#include <sstream>
#include <string>
#include <vector>

#include "twd_internal.h"

namespace twd {
namespace {

constexpr uint32_t kMagic = 0x4734444Eu;  // 'G4DN'
constexpr uint32_t kVersion = 3;          // v2 changed the layer layout and is rejected
constexpr uint64_t kAlign = 4096;
constexpr uint32_t kMaxLayers = 60;
constexpr uint32_t kQuantAffineInt4G64 = 1;
constexpr uint32_t kScaleBf16 = 1;

#pragma pack(push, 1)
struct Header {
    uint32_t magic, version, quant_type, num_layers, d_model, d_ff, num_q_heads, num_kv_heads,
        head_dim, vocab_size, sliding_window, quant_group_size, scale_dtype, tied_embeddings;
    uint64_t global_layer_mask;
    float rope_theta_local, rope_theta_global, rope_scaling, final_logit_softcapping;
    uint64_t embed_offset, embed_size, lm_head_offset, lm_head_size;
    uint64_t layer_offsets[kMaxLayers];
    uint64_t layer_sizes[kMaxLayers];
    uint8_t payload_sha256[32];
    uint8_t tail[4096 - 0x450];
};
#pragma pack(pop)
static_assert(sizeof(Header) == 4096, "the container header is 4096 bytes");
static_assert(offsetof(Header, final_logit_softcapping) == 0x4C, "header layout");
static_assert(offsetof(Header, lm_head_offset) == 0x60, "header layout");
static_assert(offsetof(Header, layer_offsets) == 0x70, "header layout");
static_assert(offsetof(Header, layer_sizes) == 0x250, "header layout");
static_assert(offsetof(Header, payload_sha256) == 0x430, "header layout");

// validate_header of src/format.cpp:6-65, with the same checks in the same order and the same
// messages; returns an empty string when the header is accepted.
std::string validate(const Header& h, uint64_t file_size) {
    std::stringstream ss;
    if (h.magic != kMagic) {
        ss << "Invalid magic: expected 0x" << std::hex << kMagic << ", got 0x" << h.magic;
        return ss.str();
    }
    if (h.version != kVersion) {
        ss << "Unsupported container version: expected " << kVersion << ", got " << h.version;
        return ss.str();
    }
    if (h.num_layers == 0 || h.num_layers > kMaxLayers) {
        ss << "Invalid layer count: " << h.num_layers << " (max " << kMaxLayers << ")";
        return ss.str();
    }
    if (h.d_model == 0 || h.d_ff == 0 || h.vocab_size == 0)
        return "Invalid model geometry dimensions (d_model, d_ff, or vocab_size is zero)";
    if (h.embed_offset % kAlign != 0) return "Embedding offset is not 4096-byte aligned";
    if (h.lm_head_offset % kAlign != 0) return "LM head offset is not 4096-byte aligned";
    for (uint32_t i = 0; i < h.num_layers; ++i) {
        if (h.layer_offsets[i] % kAlign != 0) {
            ss << "Layer " << i << " offset (" << h.layer_offsets[i] << ") is not 4096-byte aligned";
            return ss.str();
        }
        if (h.layer_sizes[i] == 0) {
            ss << "Layer " << i << " has size 0";
            return ss.str();
        }
        if (h.layer_offsets[i] + h.layer_sizes[i] < h.layer_offsets[i]) return "layer bounds: arithmetic overflow";
        if (file_size > 0 && h.layer_offsets[i] + h.layer_sizes[i] > file_size) {
            ss << "Layer " << i << " extends beyond file bounds (offset=" << h.layer_offsets[i]
               << ", size=" << h.layer_sizes[i] << ", file_size=" << file_size << ")";
            return ss.str();
        }
    }
    return std::string();
}

struct File {
    FILE* f = nullptr;
    ~File() {
        if (f) std::fclose(f);
    }
};

int open_container(const char* path, File& file, Header& h, uint64_t& size) {
    if (!path) return fail(TWD_E_INVALID, "null path");
    file.f = std::fopen(path, "rb");
    if (!file.f) return fail(TWD_E_INVALID, std::string("cannot open ") + path);
    if (std::fseek(file.f, 0, SEEK_END) != 0) return fail(TWD_E_INVALID, "cannot seek the container");
    const long end = std::ftell(file.f);
    if (end < 0) return fail(TWD_E_INVALID, "cannot size the container");
    size = static_cast<uint64_t>(end);
    if (size < sizeof(Header)) return fail(TWD_E_INVALID, "file is shorter than the 4096-byte header");
    std::rewind(file.f);
    if (std::fread(&h, sizeof(Header), 1, file.f) != 1) return fail(TWD_E_INVALID, "cannot read the header");
    const std::string err = validate(h, size);
    if (!err.empty()) return fail(TWD_E_INVALID, err);
    return TWD_OK;
}

bool read_at(FILE* f, uint64_t offset, void* dst, uint64_t n) {
    if (std::fseek(f, static_cast<long>(offset), SEEK_SET) != 0) return false;
    return std::fread(dst, 1, n, f) == n;
}

}  // namespace
}  // namespace twd

using namespace twd;

extern "C" {

TWD_API int twd_container_inspect(const char* path, twd_container_info* info) {
    clear_error();
    if (!info) return fail(TWD_E_INVALID, "null info");
    File file;
    Header h;
    uint64_t size = 0;
    int rc = open_container(path, file, h, size);
    if (rc) return rc;
    info->version = h.version;
    info->quant_type = h.quant_type;
    info->num_layers = h.num_layers;
    info->d_model = h.d_model;
    info->d_ff = h.d_ff;
    info->vocab_size = h.vocab_size;
    info->quant_group_size = h.quant_group_size;
    info->scale_dtype = h.scale_dtype;
    info->tied_embeddings = h.tied_embeddings;
    info->final_logit_softcapping = h.final_logit_softcapping;
    info->embed_offset = h.embed_offset;
    info->embed_size = h.embed_size;
    info->lm_head_offset = h.lm_head_offset;
    info->lm_head_size = h.lm_head_size;
    info->file_size = size;
    return TWD_OK;
}

TWD_API int twd_head_load(const char* path, void* stream, twd_head** out) {
    clear_error();
    if (!out) return fail(TWD_E_INVALID, "null out");
    *out = nullptr;
    File file;
    Header h;
    uint64_t size = 0;
    int rc = open_container(path, file, h, size);
    if (rc) return rc;
    if (h.quant_type != kQuantAffineInt4G64 || h.quant_group_size != 64 || h.scale_dtype != kScaleBf16)
        return fail(TWD_E_UNSUPPORTED, "the LM head must be affine INT4 with 64-wide groups and bf16 scales");
    const uint32_t V = h.vocab_size, d = h.d_model;
    if (d % kChunkK != 0) return fail(TWD_E_UNSUPPORTED, "d_model must be a multiple of 128");
    // runner.cpp:427-437: the [W|S|B] slice must fit the header's lm_head_size
    const uint64_t w_bytes = static_cast<uint64_t>(V) * (d / 8) * 4;
    const uint64_t s_bytes = static_cast<uint64_t>(V) * (d / 64) * 2;
    const uint64_t total = w_bytes + 2 * s_bytes;
    if (total > h.lm_head_size) {
        return fail(TWD_E_INVALID, "ForwardRunner: computed LM head size " + std::to_string(total) +
                                       " exceeds header lm_head_size " + std::to_string(h.lm_head_size));
    }
    if (h.lm_head_offset > size || total > size - h.lm_head_offset)
        return fail(TWD_E_INVALID, "the LM head extends beyond the file");

    // the slice, staged through a pinned chunk into a device copy of the reference layout
    const hipStream_t s = static_cast<hipStream_t>(stream);
    constexpr uint64_t kChunk = 64ull << 20;
    void* dev = nullptr;
    void* pinned = nullptr;
    TWD_HIP(hipMalloc(&dev, total));
    hipError_t e = hipHostMalloc(&pinned, std::min(kChunk, total), hipHostMallocDefault);
    if (e != hipSuccess) {
        (void)hipFree(dev);
        return hip_fail(e, "hipHostMalloc");
    }
    bool ok = true;
    for (uint64_t off = 0; ok && off < total; off += kChunk) {
        const uint64_t n = std::min(kChunk, total - off);
        ok = read_at(file.f, h.lm_head_offset + off, pinned, n);
        if (!ok) break;
        e = hipMemcpyAsync(static_cast<uint8_t*>(dev) + off, pinned, n, hipMemcpyHostToDevice, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        ok = e == hipSuccess;
    }
    (void)hipHostFree(pinned);
    if (!ok) {
        (void)hipFree(dev);
        return e != hipSuccess ? hip_fail(e, "uploading the LM head") : fail(TWD_E_INVALID, "cannot read the LM head");
    }
    twd_head* head = nullptr;
    rc = twd_head_create_device(dev, total, V, d, 64, h.final_logit_softcapping, stream, &head);
    (void)hipFree(dev);
    if (rc) return rc;

    // the final RMSNorm weight follows the embedding table's [W|S|B] (runner.cpp:488-497)
    if (h.embed_offset > 0 && h.embed_offset <= size && total <= size - h.embed_offset) {
        const uint64_t at = h.embed_offset + total;
        if (2ull * d <= size - at) {
            std::vector<uint16_t> w(d);
            if (!read_at(file.f, at, w.data(), 2ull * d)) {
                twd_head_destroy(head);
                return fail(TWD_E_INVALID, "cannot read the final norm weight");
            }
            if ((rc = head_set_norm_weight(head, w.data(), d))) {
                twd_head_destroy(head);
                return rc;
            }
        }
    }
    *out = head;
    return TWD_OK;
}

}  // extern "C"
