// wpk.cpp - the model.wpk weight package: checks and upload.
//
// Format (the reference's WPK v1, native/runtime/weight_loader.h:4-10 and
// weight_loader.cpp:21-47; little endian, packed):
//   header, 64 bytes: magic u32 = 0x31504B4D, abi_version u16 = 2,
//     target_sm u16 = 120, model_hash u8[32], section_count u32,
//     reserved u32 = 0, toc_offset u64 = 64, data_start u64;
//   TOC at toc_offset, section_count entries of 132 bytes: name_hash u64
//     (FNV-1a 64 of the UTF-8 name), dtype u32 (0 = bf16), layout u32
//     (0 = row-major [out][in]), rank u32, dims u32[8], data_offset u64,
//     data_bytes u64, scale_offset u64, scale_bytes u64, reserved u64[6].
// The package holds exactly the 3 + 42 x 6 sections of the model
// ("embedding", "lm_head", "final_norm", "layer<i>.{norm1,qkv,o,norm2,
// gate_up,down}") with the shapes of generated_model_config.h; every check
// of the reference loader (weight_loader.cpp:201-330) is made, plus that each
// section's data lies inside the file. The section data is placed in one
// device allocation at 256-byte aligned offsets and uploaded through two
// pinned 64 MiB staging buffers, so reading the next block from the file
// overlaps the copy of the previous one. The reference's layer-window
// switches (MC_LOAD_LAYERS_MIN / MAX, MC_LOAD_SKIP_EMBEDDING / LM_HEAD) are
// not supported: with one set the load fails with MC_E_UNSUPPORTED.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "error.h"
#include "model_internal.h"
#include "trace.h"

namespace mckv {
namespace {

#pragma pack(push, 1)
struct WpkHeader {
    uint32_t magic;
    uint16_t abi_version;
    uint16_t target_sm;
    uint8_t model_hash[32];
    uint32_t section_count;
    uint32_t reserved;
    uint64_t toc_offset;
    uint64_t data_start;
};
struct WpkEntry {
    uint64_t name_hash;
    uint32_t dtype;
    uint32_t layout;
    uint32_t rank;
    uint32_t dims[8];
    uint64_t data_offset;
    uint64_t data_bytes;
    uint64_t scale_offset;
    uint64_t scale_bytes;
    uint64_t reserved[6];
};
#pragma pack(pop)
static_assert(sizeof(WpkHeader) == 64, "header layout");
static_assert(sizeof(WpkEntry) == 132, "TOC entry layout");

constexpr uint32_t kMagic = 0x31504B4Du;  // "MKP1"
constexpr uint16_t kAbi = 2;
constexpr uint16_t kTargetSm = 120;
constexpr size_t kSections = 3 + (size_t)kModelLayers * 6;
constexpr size_t kStage = 64ull << 20;

uint64_t fnv1a64(const std::string& s) {
    uint64_t h = 14695981039346656037ull;
    for (unsigned char c : s) {
        h ^= c;
        h *= 1099511628211ull;
    }
    return h;
}

// One section the model needs: name, shape, and where its pointer goes.
struct Want {
    std::string name;
    uint32_t rank;
    uint32_t dims[2];
    const uint16_t** slot;  // in ModelWeights (nullptr when only checking)
};

std::vector<Want> wanted(ModelWeights* w) {
    std::vector<Want> v;
    auto at = [&](const uint16_t** p) { return w != nullptr ? p : nullptr; };
    v.push_back({"embedding", 2, {kVocabSize, kHidden}, at(w ? &w->embedding : nullptr)});
    v.push_back({"lm_head", 2, {kVocabSize, kHidden}, at(w ? &w->lm_head : nullptr)});
    v.push_back({"final_norm", 1, {kHidden, 0}, at(w ? &w->final_norm : nullptr)});
    for (uint32_t i = 0; i < kModelLayers; ++i) {
        const std::string p = "layer" + std::to_string(i) + ".";
        v.push_back({p + "norm1", 1, {kHidden, 0}, at(w ? &w->norm1[i] : nullptr)});
        v.push_back({p + "qkv", 2, {kQkvCols, kHidden}, at(w ? &w->qkv[i] : nullptr)});
        v.push_back({p + "o", 2, {kHidden, kHidden}, at(w ? &w->o[i] : nullptr)});
        v.push_back({p + "norm2", 1, {kHidden, 0}, at(w ? &w->norm2[i] : nullptr)});
        v.push_back({p + "gate_up", 2, {2 * kInter, kHidden}, at(w ? &w->gate_up[i] : nullptr)});
        v.push_back({p + "down", 2, {kHidden, kInter}, at(w ? &w->down[i] : nullptr)});
    }
    return v;
}

struct File {
    FILE* f = nullptr;
    ~File() {
        if (f) std::fclose(f);
    }
};

bool read_at(FILE* f, uint64_t off, void* dst, size_t n) {
    if (fseeko(f, (off_t)off, SEEK_SET) != 0) return false;
    return std::fread(dst, 1, n, f) == n;
}

struct Pinned {
    void* p[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    ~Pinned() {
        for (int i = 0; i < 2; ++i) {
            if (ev[i]) {
                (void)hipEventSynchronize(ev[i]);
                (void)hipEventDestroy(ev[i]);
            }
            if (p[i]) (void)hipHostFree(p[i]);
        }
    }
};

// One contiguous piece of the file and where it goes in a device allocation.
struct Piece {
    uint64_t file_off, bytes, arena_off;
    const char* what;  // section name, for error messages
};

// Uploads the pieces through two pinned 64 MiB staging buffers (reading the
// next block from the file overlaps the copy of the previous one). On error
// the stream is synchronized (no copy still targets the allocation) and the
// error set.
mc_status_t upload(FILE* f, const std::vector<Piece>& pieces, char* arena, hipStream_t st,
                   const char* pkg) {
    Pinned pin;
    hipError_t he = hipSuccess;
    for (int b = 0; b < 2 && he == hipSuccess; ++b) {
        he = hipHostMalloc(&pin.p[b], kStage);
        if (he == hipSuccess) he = hipEventCreateWithFlags(&pin.ev[b], hipEventDisableTiming);
    }
    if (he != hipSuccess) return check_hip(he, "weight package: staging buffers");
    int b = 0;
    bool used[2] = {false, false};
    for (const Piece& pc : pieces) {
        for (uint64_t done = 0; done < pc.bytes && he == hipSuccess;) {
            const size_t n = (size_t)std::min<uint64_t>(kStage, pc.bytes - done);
            if (used[b]) {
                he = hipEventSynchronize(pin.ev[b]);  // staging buffer b is free again
                if (he != hipSuccess) break;
            }
            if (!read_at(f, pc.file_off + done, pin.p[b], n)) {
                (void)hipStreamSynchronize(st);  // copies in flight still target the arena
                set_error("%s: read of section '%s' failed", pkg, pc.what);
                return MC_E_IO;
            }
            he = hipMemcpyAsync(arena + pc.arena_off + done, pin.p[b], n, hipMemcpyHostToDevice,
                                st);
            if (he == hipSuccess) he = hipEventRecord(pin.ev[b], st);
            used[b] = true;
            b ^= 1;
            done += n;
        }
        if (he != hipSuccess) break;
    }
    if (he == hipSuccess) he = hipStreamSynchronize(st);
    if (he != hipSuccess) {
        (void)hipStreamSynchronize(st);
        return check_hip(he, "weight package upload");
    }
    return MC_OK;
}

// Header checks shared by both packages (weight_loader.cpp:201-230,497-507).
mc_status_t read_header(FILE* f, const char* path, uint64_t fsize, const char* pkg,
                        WpkHeader* h, std::vector<WpkEntry>* toc) {
    if (!read_at(f, 0, h, sizeof(*h))) {
        set_error("%s: '%s' is shorter than its 64-byte header", pkg, path);
        return MC_E_IO;
    }
    if (h->magic != kMagic || h->abi_version != kAbi || h->target_sm != kTargetSm) {
        set_error("%s: header magic/abi/target 0x%08x/%u/%u, expected 0x%08x/%u/%u", pkg,
                  h->magic, h->abi_version, h->target_sm, kMagic, kAbi, kTargetSm);
        return MC_E_MODEL_MISMATCH;
    }
    if (h->toc_offset != 64u || h->reserved != 0u || h->section_count == 0u ||
        h->data_start > fsize ||
        (uint64_t)h->section_count * sizeof(WpkEntry) > h->data_start - h->toc_offset) {
        set_error("%s: inconsistent header (toc_offset %llu, reserved %u, %u sections, "
                  "data_start %llu, file %llu bytes)",
                  pkg, (unsigned long long)h->toc_offset, h->reserved, h->section_count,
                  (unsigned long long)h->data_start, (unsigned long long)fsize);
        return MC_E_MODEL_MISMATCH;
    }
    toc->resize(h->section_count);
    if (!read_at(f, h->toc_offset, toc->data(), toc->size() * sizeof(WpkEntry))) {
        set_error("%s: cannot read the %u-entry section table", pkg, h->section_count);
        return MC_E_IO;
    }
    return MC_OK;
}

}  // namespace

void wpk_free(ModelWeights* w) {
    if (w == nullptr) return;
    if (w->arena) (void)hipFree(w->arena);
    if (w->fp8_arena) (void)hipFree(w->fp8_arena);
    *w = ModelWeights{};
}

mc_status_t wpk_load(const char* path, ModelWeights* w, uint64_t* arena_bytes, hipStream_t st) {
    TraceRange trace_range("wpk_load");
    if (w != nullptr) *w = ModelWeights{};
    for (const char* env : {"MC_LOAD_LAYERS_MIN", "MC_LOAD_LAYERS_MAX", "MC_LOAD_SKIP_EMBEDDING",
                            "MC_LOAD_SKIP_LM_HEAD"}) {
        const char* v = std::getenv(env);
        if (v != nullptr && v[0] != '\0') {
            set_error("model.wpk: %s is set; this build loads whole models only", env);
            return MC_E_UNSUPPORTED;
        }
    }
    File file;
    file.f = std::fopen(path, "rb");
    if (file.f == nullptr) {
        set_error("model.wpk: cannot open '%s'", path);
        return MC_E_IO;
    }
    if (fseeko(file.f, 0, SEEK_END) != 0) {
        set_error("model.wpk: cannot seek in '%s'", path);
        return MC_E_IO;
    }
    const uint64_t fsize = (uint64_t)ftello(file.f);
    WpkHeader h{};
    std::vector<WpkEntry> toc;
    if (const mc_status_t rs = read_header(file.f, path, fsize, "model.wpk", &h, &toc);
        rs != MC_OK)
        return rs;
    std::unordered_map<uint64_t, const WpkEntry*> by_hash;
    for (const WpkEntry& e : toc)
        if (!by_hash.emplace(e.name_hash, &e).second) {
            set_error("model.wpk: two sections share the name hash 0x%016llx",
                      (unsigned long long)e.name_hash);
            return MC_E_MODEL_MISMATCH;
        }
    if (by_hash.size() != kSections) {
        set_error("model.wpk: %zu sections, the model has %zu", by_hash.size(), kSections);
        return MC_E_MODEL_MISMATCH;
    }
    std::vector<Want> want = wanted(w);
    std::vector<const WpkEntry*> found(want.size());
    std::vector<uint64_t> place(want.size());
    uint64_t cursor = 0;
    for (size_t i = 0; i < want.size(); ++i) {
        const Want& q = want[i];
        const auto it = by_hash.find(fnv1a64(q.name));
        if (it == by_hash.end()) {
            set_error("model.wpk: section '%s' is missing", q.name.c_str());
            return MC_E_MODEL_MISMATCH;
        }
        const WpkEntry& e = *it->second;
        uint64_t elems = 1;
        bool dims_ok = e.rank == q.rank;
        for (uint32_t d = 0; dims_ok && d < q.rank; ++d) {
            dims_ok = e.dims[d] == q.dims[d];
            elems *= q.dims[d];
        }
        if (e.dtype != 0u || e.layout != 0u || !dims_ok) {
            set_error("model.wpk: section '%s' is not a bf16 row-major tensor of the model's "
                      "shape (dtype %u, layout %u, rank %u)",
                      q.name.c_str(), e.dtype, e.layout, e.rank);
            return MC_E_MODEL_MISMATCH;
        }
        if (e.data_bytes != elems * 2u || e.data_offset < h.data_start ||
            e.data_offset > fsize || e.data_bytes > fsize - e.data_offset) {
            set_error("model.wpk: section '%s' holds %llu bytes at offset %llu; expected %llu "
                      "bytes inside the data area of the %llu-byte file",
                      q.name.c_str(), (unsigned long long)e.data_bytes,
                      (unsigned long long)e.data_offset, (unsigned long long)(elems * 2u),
                      (unsigned long long)fsize);
            return MC_E_MODEL_MISMATCH;
        }
        found[i] = &e;
        cursor = (cursor + 255u) & ~uint64_t(255);
        place[i] = cursor;
        cursor += e.data_bytes;
    }
    if (arena_bytes != nullptr) *arena_bytes = cursor;
    if (w == nullptr) return MC_OK;

    hipError_t he = hipMalloc(&w->arena, cursor);
    if (he != hipSuccess) {
        (void)hipGetLastError();
        w->arena = nullptr;
        set_error("model.wpk: cannot allocate %llu bytes of device memory for the weights",
                  (unsigned long long)cursor);
        return MC_E_OUT_OF_MEMORY;
    }
    w->bytes = cursor;
    std::vector<Piece> pieces;
    for (size_t i = 0; i < want.size(); ++i)
        pieces.push_back({found[i]->data_offset, found[i]->data_bytes, place[i],
                          want[i].name.c_str()});
    if (const mc_status_t rs = upload(file.f, pieces, static_cast<char*>(w->arena), st,
                                      "model.wpk");
        rs != MC_OK) {
        wpk_free(w);
        return rs;
    }
    for (size_t i = 0; i < want.size(); ++i)
        *want[i].slot = reinterpret_cast<const uint16_t*>(static_cast<char*>(w->arena) + place[i]);
    return MC_OK;
}

mc_status_t wpk_load_fp8(const char* path, ModelWeights* w, uint64_t* arena_bytes,
                         hipStream_t st) {
    TraceRange trace_range("wpk_load_fp8");
    const char* pkg = "model_fp8.wpk";
    File file;
    file.f = std::fopen(path, "rb");
    if (file.f == nullptr) {
        set_error("%s: cannot open '%s' (precision MC_FP8 needs it beside model.wpk)", pkg,
                  path);
        return MC_E_MODEL_MISMATCH;
    }
    if (fseeko(file.f, 0, SEEK_END) != 0) {
        set_error("%s: cannot seek in '%s'", pkg, path);
        return MC_E_IO;
    }
    const uint64_t fsize = (uint64_t)ftello(file.f);
    WpkHeader h{};
    std::vector<WpkEntry> toc;
    if (const mc_status_t rs = read_header(file.f, path, fsize, pkg, &h, &toc); rs != MC_OK)
        return rs;
    std::unordered_map<uint64_t, const WpkEntry*> by_hash;
    for (const WpkEntry& e : toc)
        if (!by_hash.emplace(e.name_hash, &e).second) {
            set_error("%s: two sections share the name hash 0x%016llx", pkg,
                      (unsigned long long)e.name_hash);
            return MC_E_MODEL_MISMATCH;
        }
    // the 42 x 4 quantized projections, then the lm_head when the package
    // has a dtype-2 one and MC_FP8_LMHEAD_OFF is unset (weight_loader.cpp:
    // 525-560); other sections are ignored
    struct Q {
        std::string name;
        uint32_t rows, cols;
        const uint8_t** q;
        const float** s;
    };
    std::vector<Q> want;
    ModelWeights dummy;
    ModelWeights& d = w != nullptr ? *w : dummy;
    for (uint32_t i = 0; i < kModelLayers; ++i) {
        const std::string p = "layer" + std::to_string(i) + ".";
        want.push_back({p + "qkv", kQkvCols, kHidden, &d.q_qkv[i], &d.s_qkv[i]});
        want.push_back({p + "o", kHidden, kHidden, &d.q_o[i], &d.s_o[i]});
        want.push_back({p + "gate_up", 2 * kInter, kHidden, &d.q_gate_up[i], &d.s_gate_up[i]});
        want.push_back({p + "down", kHidden, kInter, &d.q_down[i], &d.s_down[i]});
    }
    if (std::getenv("MC_FP8_LMHEAD_OFF") == nullptr) {
        const auto it = by_hash.find(fnv1a64("lm_head"));
        if (it != by_hash.end() && it->second->dtype == 2u)
            want.push_back({"lm_head", kVocabSize, kHidden, &d.q_lm_head, &d.s_lm_head});
    }
    std::vector<Piece> pieces;
    std::vector<uint64_t> qoff(want.size()), soff(want.size());
    uint64_t cursor = 0;
    for (size_t i = 0; i < want.size(); ++i) {
        const Q& q = want[i];
        const auto it = by_hash.find(fnv1a64(q.name));
        if (it == by_hash.end()) {
            set_error("%s: quantized section '%s' is missing", pkg, q.name.c_str());
            return MC_E_MODEL_MISMATCH;
        }
        const WpkEntry& e = *it->second;
        if (e.dtype != 2u || e.layout != 0u || e.rank != 2u || e.dims[0] != q.rows ||
            e.dims[1] != q.cols) {
            set_error("%s: section '%s' is not an e4m3 row-major [%u][%u] tensor (dtype %u, "
                      "layout %u, rank %u, dims %u x %u)",
                      pkg, q.name.c_str(), q.rows, q.cols, e.dtype, e.layout, e.rank, e.dims[0],
                      e.dims[1]);
            return MC_E_MODEL_MISMATCH;
        }
        const uint64_t db = (uint64_t)q.rows * q.cols, sb = (uint64_t)q.rows * 4u;
        if (e.data_bytes != db || e.scale_bytes != sb || e.data_offset < h.data_start ||
            e.scale_offset < h.data_start || e.data_offset > fsize ||
            e.data_bytes > fsize - e.data_offset || e.scale_offset > fsize ||
            e.scale_bytes > fsize - e.scale_offset) {
            set_error("%s: section '%s' holds %llu + %llu bytes at %llu / %llu; expected %llu "
                      "code and %llu scale bytes inside the %llu-byte file",
                      pkg, q.name.c_str(), (unsigned long long)e.data_bytes,
                      (unsigned long long)e.scale_bytes, (unsigned long long)e.data_offset,
                      (unsigned long long)e.scale_offset, (unsigned long long)db,
                      (unsigned long long)sb, (unsigned long long)fsize);
            return MC_E_MODEL_MISMATCH;
        }
        qoff[i] = cursor;
        cursor = (cursor + db + 255u) & ~uint64_t(255);
        soff[i] = cursor;
        cursor = (cursor + sb + 255u) & ~uint64_t(255);
        pieces.push_back({e.data_offset, db, qoff[i], q.name.c_str()});
        pieces.push_back({e.scale_offset, sb, soff[i], q.name.c_str()});
    }
    if (arena_bytes != nullptr) *arena_bytes = cursor;
    if (w == nullptr) return MC_OK;
    if (hipMalloc(&w->fp8_arena, cursor) != hipSuccess) {
        (void)hipGetLastError();
        w->fp8_arena = nullptr;
        set_error("%s: cannot allocate %llu bytes of device memory", pkg,
                  (unsigned long long)cursor);
        return MC_E_OUT_OF_MEMORY;
    }
    w->fp8_bytes = cursor;
    char* base = static_cast<char*>(w->fp8_arena);
    if (const mc_status_t rs = upload(file.f, pieces, base, st, pkg); rs != MC_OK) {
        (void)hipFree(w->fp8_arena);
        w->fp8_arena = nullptr;
        w->fp8_bytes = 0;
        return rs;
    }
    for (size_t i = 0; i < want.size(); ++i) {
        *want[i].q = reinterpret_cast<const uint8_t*>(base + qoff[i]);
        *want[i].s = reinterpret_cast<const float*>(base + soff[i]);
    }
    return MC_OK;
}

}  // namespace mckv

extern "C" mc_status_t mc_model_wpk_check(const char* path, uint64_t* arena_bytes) {
    if (path == nullptr || arena_bytes == nullptr) {
        mckv::set_error("mc_model_wpk_check: path or arena_bytes is NULL");
        return MC_E_INVALID_ARGUMENT;
    }
    MC_GUARD_BEGIN
    return mckv::wpk_load(path, nullptr, arena_bytes, nullptr);
    MC_GUARD_END
}

extern "C" mc_status_t mc_model_wpk_fp8_check(const char* path, uint64_t* arena_bytes) {
    if (path == nullptr || arena_bytes == nullptr) {
        mckv::set_error("mc_model_wpk_fp8_check: path or arena_bytes is NULL");
        return MC_E_INVALID_ARGUMENT;
    }
    MC_GUARD_BEGIN
    return mckv::wpk_load_fp8(path, nullptr, arena_bytes, nullptr);
    MC_GUARD_END
}
