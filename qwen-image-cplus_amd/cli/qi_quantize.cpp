// qi-quantize: writes and verifies INT4 transformer packs, the command of
// qwen_image_quantize/src/main.cplus:9-55 with the same arguments:
//
//   qi-quantize w4a16|w4a4 SOURCE_FP16_QIPACK OUTPUT [GROUP] [clip]
//   qi-quantize verify FILE
//
// The source is the all-FP16 v4 QIPACK (policy transformer:all-matrix-f16-v4,
// 297 records).  Every rank-2 FP16 record (the 224 block matrices) becomes an
// INT4 record of the chosen scheme; every other record is copied byte for
// byte (int4_pack.cplus:472-518, 542-731).  The quantisers run on the GPU
// through qi_hip_pack_weights (bit-exact to int4_pack.cplus:237-468), one
// matrix at a time.  The output is written to OUTPUT.tmp, verified with the
// packer's verify (qi_pack_verify, int4_pack.cplus:733-850) and renamed.
//
// GROUP: the reference accepts 32, 64, 128 and 256, but its engine loads
// only g64 packs (transformer.cplus:312-313, 353-356); this build packs
// group 64 and rejects the others with exit status 2, as it does a group
// that does not divide 256.
//
// Exit status: 0 success, 1 failure, 2 usage (as main.cplus:9-13).

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/qwen_image_hip.h"

namespace {

constexpr uint64_t kFnvOffset = 14695981039346656037ull;
constexpr uint64_t kAlign = 256;
constexpr uint32_t kTensorCount = 297, kBlockMatrices = 224;
constexpr uint32_t kSchemeFp16 = 1, kSchemeW4A16 = 5, kSchemeW4A4 = 6;
constexpr uint32_t kTypeNone = 0, kTypeF16 = 1, kMetadataVersion = 1;
constexpr const char *kSourcePolicy = "transformer:all-matrix-f16-v4";

// The 256-byte little-endian header and record (int4_pack.cplus:55-95).
#pragma pack(push, 1)
struct Header {
    uint8_t magic[8];
    uint32_t version, header_bytes, tensor_count, scope;
    uint64_t directory_offset, data_offset, file_bytes, payload_checksum;
    uint8_t model_snapshot[40], diffusers_commit[40], policy[32];
    uint64_t metadata_offset;
    uint32_t metadata_bytes, metadata_version;
    uint64_t metadata_checksum;
    uint8_t reserved[64];
};
struct Record {
    char name[128];
    uint32_t scheme, rank;
    uint64_t dims[4];
    uint32_t group_axis, group_size, scale_type, zero_type;
    uint64_t weights_offset, weights_length, scales_offset, scales_length, zeros_offset, zeros_length;
    uint64_t elements, tensor_checksum;
    uint8_t reserved[8];
};
#pragma pack(pop)
static_assert(sizeof(Header) == 256 && offsetof(Header, policy) == 136 && offsetof(Header, metadata_offset) == 168,
              "QIPACK1 header layout");
static_assert(sizeof(Record) == 256 && offsetof(Record, weights_offset) == 184 && offsetof(Record, elements) == 232,
              "QIPACK1 record layout");

int usage() {
    std::fprintf(stderr, "usage: qi-quantize w4a16|w4a4 SOURCE_FP16_QIPACK OUTPUT [GROUP] [clip]\n");
    std::fprintf(stderr, "       qi-quantize verify FILE\n");
    return 2;
}

uint64_t align_up(uint64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

bool io_at(int fd, void *buf, uint64_t length, uint64_t offset, bool write) {
    uint8_t *p = static_cast<uint8_t *>(buf);
    while (length) {
        const size_t step = length > (1ull << 30) ? (1ull << 30) : static_cast<size_t>(length);
        const ssize_t done = write ? pwrite(fd, p, step, static_cast<off_t>(offset))
                                   : pread(fd, p, step, static_cast<off_t>(offset));
        if (done <= 0) return false;
        p += done;
        offset += static_cast<uint64_t>(done);
        length -= static_cast<uint64_t>(done);
    }
    return true;
}

bool fixed_equals(const uint8_t *field, size_t capacity, const char *text) {
    const size_t n = std::strlen(text);
    if (n > capacity) return false;
    for (size_t i = 0; i < capacity; ++i)
        if (field[i] != (i < n ? static_cast<uint8_t>(text[i]) : 0)) return false;
    return true;
}

bool fixed_set(uint8_t *field, size_t capacity, const std::string &text) {
    if (text.size() > capacity) return false;
    std::memset(field, 0, capacity);
    std::memcpy(field, text.data(), text.size());
    return true;
}

bool is_block_matrix(const Record &r) { return r.scheme == kSchemeFp16 && r.rank == 2; }

// Record of the output pack for one source record, placed at `cursor`
// (int4_pack.cplus:476-518).
Record plan_record(const Record &src, uint32_t scheme, int group, uint64_t &cursor) {
    Record r = src;
    r.tensor_checksum = 0;
    r.scales_offset = r.scales_length = r.zeros_offset = r.zeros_length = 0;
    if (is_block_matrix(src)) {
        const uint64_t n = src.dims[0], k = src.dims[1], groups = n * (k / static_cast<uint64_t>(group));
        r.scheme = scheme;
        r.group_axis = 1;
        r.group_size = static_cast<uint32_t>(group);
        r.scale_type = kTypeF16;
        r.zero_type = scheme == kSchemeW4A16 ? kTypeF16 : kTypeNone;
        r.weights_length = n * k / 2;
        r.scales_length = groups * 2;
        if (scheme == kSchemeW4A16) r.zeros_length = groups * 2;
    }
    cursor = align_up(cursor);
    r.weights_offset = cursor;
    cursor += r.weights_length;
    if (r.scales_length) {
        cursor = align_up(cursor);
        r.scales_offset = cursor;
        cursor += r.scales_length;
    }
    if (r.zeros_length) {
        cursor = align_up(cursor);
        r.zeros_offset = cursor;
        cursor += r.zeros_length;
    }
    return r;
}

// Device buffers for one matrix at a time, grown to the largest.
struct DeviceScratch {
    void *w = nullptr, *codes = nullptr, *scales = nullptr, *mins = nullptr;
    size_t w_bytes = 0;
    ~DeviceScratch() { release(); }
    void release() {
        for (void *p : {w, codes, scales, mins})
            if (p) (void)hipFree(p);
        w = codes = scales = mins = nullptr;
        w_bytes = 0;
    }
    bool reserve(size_t weight_bytes) {
        if (weight_bytes <= w_bytes) return true;
        release();
        // codes n k / 2, scales and minimums n k / 64 fp16 each: all within
        // the fp16 matrix's n k * 2 bytes.
        if (hipMalloc(&w, weight_bytes) != hipSuccess || hipMalloc(&codes, weight_bytes / 4) != hipSuccess ||
            hipMalloc(&scales, weight_bytes / 32 + 256) != hipSuccess ||
            hipMalloc(&mins, weight_bytes / 32 + 256) != hipSuccess)
            return false;
        w_bytes = weight_bytes;
        return true;
    }
};

// Quantise or copy one record into the output (int4_pack.cplus:682-731).
bool write_tensor(int src_fd, int out_fd, const Record &src, Record &out, uint32_t scheme, int clip,
                  DeviceScratch &dev) {
    std::vector<uint8_t> input(src.weights_length);
    if (!io_at(src_fd, input.data(), input.size(), src.weights_offset, false)) return false;
    if (!is_block_matrix(src)) {
        out.tensor_checksum = qi_fnv1a(kFnvOffset, input.data(), input.size());
        return io_at(out_fd, input.data(), input.size(), out.weights_offset, true);
    }
    const uint64_t n = src.dims[0], k = src.dims[1];
    if (src.weights_length != n * k * 2 || n > 0x7fffffffu || k > 0x7fffffffu) return false;
    if (!dev.reserve(input.size())) return false;
    std::vector<uint8_t> codes(out.weights_length), scales(out.scales_length), mins(out.zeros_length);
    if (hipMemcpy(dev.w, input.data(), input.size(), hipMemcpyHostToDevice) != hipSuccess) return false;
    if (qi_hip_pack_weights(dev.w, dev.codes, dev.scales, scheme == kSchemeW4A16 ? dev.mins : nullptr,
                            static_cast<int>(n), static_cast<int>(k), static_cast<int>(scheme), clip,
                            nullptr) != 0)
        return false;
    if (hipMemcpy(codes.data(), dev.codes, codes.size(), hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(scales.data(), dev.scales, scales.size(), hipMemcpyDeviceToHost) != hipSuccess)
        return false;
    if (!mins.empty() && hipMemcpy(mins.data(), dev.mins, mins.size(), hipMemcpyDeviceToHost) != hipSuccess)
        return false;
    uint64_t h = qi_fnv1a(kFnvOffset, codes.data(), codes.size());
    h = qi_fnv1a(h, scales.data(), scales.size());
    if (!mins.empty()) h = qi_fnv1a(h, mins.data(), mins.size());
    out.tensor_checksum = h;
    bool ok = io_at(out_fd, codes.data(), codes.size(), out.weights_offset, true) &&
              io_at(out_fd, scales.data(), scales.size(), out.scales_offset, true);
    if (!mins.empty()) ok = ok && io_at(out_fd, mins.data(), mins.size(), out.zeros_offset, true);
    return ok;
}

int verify_file(const char *path, bool quiet) {
    qi_pack *pack = nullptr;
    int rc = qi_pack_open(path, &pack);
    if (rc == QI_PACK_OK) rc = qi_pack_verify(pack, 1);
    qi_pack_close(pack);
    if (rc != QI_PACK_OK) {
        if (!quiet) std::fprintf(stderr, "qi-quantize: %s failed verification (status %d)\n", path, rc);
        return 1;
    }
    if (!quiet) std::printf("qi-quantize: %s verified\n", path);
    return 0;
}

int write_pack(const char *source_path, const std::string &output_path, uint32_t scheme, int group, bool clip) {
    const int src_fd = open(source_path, O_RDONLY | O_CLOEXEC);
    if (src_fd < 0) {
        std::fprintf(stderr, "qi-quantize: could not open %s\n", source_path);
        return 1;
    }
    struct Closer {
        int fd;
        ~Closer() {
            if (fd >= 0) close(fd);
        }
    } src_close{src_fd};

    Header header;
    static const uint8_t kMagic[8] = {'Q', 'I', 'P', 'A', 'C', 'K', '1', 0};
    if (!io_at(src_fd, &header, sizeof header, 0, false)) {
        std::fprintf(stderr, "qi-quantize: could not read the source header\n");
        return 1;
    }
    if (std::memcmp(header.magic, kMagic, 8) != 0 || header.tensor_count != kTensorCount ||
        !fixed_equals(header.policy, 32, kSourcePolicy)) {
        std::fprintf(stderr, "qi-quantize: the source must be an all-matrix FP16 v4 QIPACK\n");
        return 1;
    }
    const uint64_t directory_end = header.directory_offset + sizeof(Record) * kTensorCount;
    std::vector<Record> source(kTensorCount);
    if (!io_at(src_fd, source.data(), sizeof(Record) * kTensorCount, header.directory_offset, false)) {
        std::fprintf(stderr, "qi-quantize: could not read the tensor directory\n");
        return 1;
    }

    // Metadata: the source's lines plus the quantisation (int4_pack.cplus:563-580).
    std::string metadata(header.metadata_bytes, '\0');
    if (header.metadata_bytes && !io_at(src_fd, &metadata[0], metadata.size(), header.metadata_offset, false))
        return 1;
    const std::string base = scheme == kSchemeW4A16 ? "w4a16-g" + std::to_string(group)
                                                    : "w4a4-h256-g" + std::to_string(group);
    metadata += "quant=" + base + (clip ? "-clip" : "") + "\n";
    metadata += std::string("quant_source=") + kSourcePolicy + "\n";
    if (directory_end + metadata.size() > header.data_offset) {
        std::fprintf(stderr, "qi-quantize: metadata does not fit in the directory padding\n");
        return 1;
    }

    std::vector<Record> records(kTensorCount);
    uint64_t cursor = header.data_offset;
    uint32_t matrices = 0;
    for (uint32_t i = 0; i < kTensorCount; ++i) {
        if (is_block_matrix(source[i])) {
            if (source[i].dims[1] % 256 != 0) {
                std::fprintf(stderr, "qi-quantize: matrix %u input width is not a multiple of 256\n", i);
                return 1;
            }
            ++matrices;
        }
        records[i] = plan_record(source[i], scheme, group, cursor);
    }
    if (matrices != kBlockMatrices) {
        std::fprintf(stderr, "qi-quantize: expected %u FP16 block matrices, found %u\n", kBlockMatrices, matrices);
        return 1;
    }
    const uint64_t file_bytes = align_up(cursor);

    const std::string tmp = output_path + ".tmp";
    const int fd = open(tmp.c_str(), O_RDWR | O_CREAT | O_TRUNC | O_CLOEXEC, 0644);
    if (fd < 0) {
        std::fprintf(stderr, "qi-quantize: could not create %s\n", tmp.c_str());
        return 1;
    }
    bool ok = ftruncate(fd, static_cast<off_t>(file_bytes)) == 0;
    {
        DeviceScratch dev;
        for (uint32_t i = 0; ok && i < kTensorCount; ++i) {
            ok = write_tensor(src_fd, fd, source[i], records[i], scheme, clip ? 1 : 0, dev);
            if (ok && i >= 9 && (i - 9) % 9 == 8) std::printf("qi-quantize: block %u/32\n", (i - 9) / 9 + 1);
        }
    }
    // Payload checksum over the data section as written, padding included.
    uint64_t payload = kFnvOffset;
    if (ok) {
        std::vector<uint8_t> chunk(64u << 20);
        for (uint64_t pos = header.data_offset; ok && pos < file_bytes;) {
            const uint64_t amount = file_bytes - pos < chunk.size() ? file_bytes - pos : chunk.size();
            ok = io_at(fd, chunk.data(), amount, pos, false);
            payload = qi_fnv1a(payload, chunk.data(), amount);
            pos += amount;
        }
    }
    Header out = header;
    const std::string policy = scheme == kSchemeW4A16 ? "transformer:w4a16-g" + std::to_string(group) + "-v6"
                                                      : "transformer:w4a4-h256-g" + std::to_string(group) + "-v6";
    ok = ok && fixed_set(out.policy, 32, policy);
    out.file_bytes = file_bytes;
    out.payload_checksum = payload;
    out.metadata_offset = directory_end;
    out.metadata_bytes = static_cast<uint32_t>(metadata.size());
    out.metadata_version = kMetadataVersion;
    out.metadata_checksum = qi_fnv1a(kFnvOffset, metadata.data(), metadata.size());
    ok = ok && io_at(fd, &out, sizeof out, 0, true);
    ok = ok && io_at(fd, records.data(), sizeof(Record) * kTensorCount, header.directory_offset, true);
    ok = ok && io_at(fd, metadata.data(), metadata.size(), directory_end, true);
    ok = ok && fsync(fd) == 0;
    close(fd);
    if (!ok || verify_file(tmp.c_str(), true) != 0) {
        unlink(tmp.c_str());
        std::fprintf(stderr, "qi-quantize: writing or verifying %s failed\n", tmp.c_str());
        return 1;
    }
    if (rename(tmp.c_str(), output_path.c_str()) != 0) {
        unlink(tmp.c_str());
        std::fprintf(stderr, "qi-quantize: could not install %s\n", output_path.c_str());
        return 1;
    }
    std::printf("qi-quantize: wrote %s (%s, %llu bytes)\n", output_path.c_str(), policy.c_str(),
                static_cast<unsigned long long>(file_bytes));
    return 0;
}

}  // namespace

int main(int argc, char **argv) {
    if (argc < 2) return usage();
    const std::string command = argv[1];
    if (command == "verify") {
        if (argc < 3) return usage();
        return verify_file(argv[2], false);
    }
    uint32_t scheme;
    if (command == "w4a16")
        scheme = kSchemeW4A16;
    else if (command == "w4a4")
        scheme = kSchemeW4A4;
    else
        return usage();
    if (argc < 4) return usage();
    int group = 64;
    bool clip = false;
    for (int i = 4; i < argc; ++i) {
        const std::string a = argv[i];
        if (a == "clip")
            clip = true;
        else if (a == "32" || a == "64" || a == "128" || a == "256")
            group = std::stoi(a);
        else
            return usage();
    }
    if (group != 64) {
        std::fprintf(stderr,
                     "qi-quantize: group %d: this build writes g64 packs only, the group size the engine loads\n",
                     group);
        return 2;
    }
    return write_pack(argv[2], argv[3], scheme, group, clip);
}
