// QIPACK1 container, host side: open, record lookup, ranged reads and the
// integrity check, so an engine can verify a pack and hand each INT4
// record's arrays to the device re-layout (qi_hip_relayout_w4a4_fp6 /
// qi_hip_relayout_w4a16) at upload.
//
// Format: qwen_image_cuda/src/int4_pack.cplus:55-95 (256-byte header and
// records, little-endian, tensors on 256-byte boundaries :36-38).  Checks:
// the reference loader's header / policy test (transformer.cplus:342-375)
// and its packer's verify (int4_pack.cplus:733-850): INT4 record geometry,
// monotonic aligned tensor placement inside the data section, metadata,
// per-tensor and payload FNV-1a 64 checksums (int4_pack.cplus:151-159).

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <new>
#include <vector>

#include "../../include/qwen_image_hip.h"

#define QI_PACK_API extern "C" __attribute__((visibility("default")))

namespace {

constexpr uint64_t kFnvOffset = 14695981039346656037ull;
constexpr uint64_t kFnvPrime = 1099511628211ull;
constexpr uint64_t kHeaderBytes = 256, kRecordBytes = 256, kAlign = 256;
constexpr uint32_t kSchemeBf16 = 0, kSchemeFp16 = 1, kSchemeW4A16 = 5, kSchemeW4A4 = 6;

uint64_t fnv1a(uint64_t h, const uint8_t *p, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) h = (h ^ p[i]) * kFnvPrime;
    return h;
}

template <typename T>
T load_le(const uint8_t *p) {  // the container is little-endian, as is the host
    T v;
    std::memcpy(&v, p, sizeof(T));
    return v;
}

bool read_at(int fd, void *dst, uint64_t length, uint64_t offset) {
    uint8_t *out = static_cast<uint8_t *>(dst);
    while (length) {
        const ssize_t got = pread(fd, out, length > (1u << 30) ? (1u << 30) : length, static_cast<off_t>(offset));
        if (got <= 0) return false;
        out += got;
        offset += static_cast<uint64_t>(got);
        length -= static_cast<uint64_t>(got);
    }
    return true;
}

// Hash `length` bytes of the file from `offset` in 8 MiB pieces.
bool hash_range(int fd, uint64_t offset, uint64_t length, uint64_t &h, std::vector<uint8_t> &chunk) {
    while (length) {
        const uint64_t n = length < chunk.size() ? length : chunk.size();
        if (!read_at(fd, chunk.data(), n, offset)) return false;
        h = fnv1a(h, chunk.data(), n);
        offset += n;
        length -= n;
    }
    return true;
}

int scheme_of_policy(const char *policy) {
    static const char *const w4a16[] = {"transformer:w4a16-g64-v6", "transformer:w4a16-g128-v6",
                                        "transformer:w4a16-g32-v6"};
    static const char *const w4a4[] = {"transformer:w4a4-h256-g64-v6", "transformer:w4a4-h256-g128-v6",
                                       "transformer:w4a4-h256-g32-v6"};
    for (const char *p : w4a16)
        if (!std::strcmp(policy, p)) return kSchemeW4A16;
    for (const char *p : w4a4)
        if (!std::strcmp(policy, p)) return kSchemeW4A4;
    return -1;
}

}  // namespace

struct qi_pack {
    int fd = -1;
    uint32_t tensor_count = 0;
    uint64_t directory_offset = 0, data_offset = 0, file_bytes = 0, payload_checksum = 0;
    uint64_t metadata_offset = 0, metadata_checksum = 0;
    uint32_t metadata_bytes = 0;
    char policy[33] = {0};
    std::vector<qi_pack_record> records;
};

QI_PACK_API uint64_t qi_fnv1a(uint64_t hash, const void *bytes, uint64_t count) {
    return fnv1a(hash, static_cast<const uint8_t *>(bytes), count);
}

QI_PACK_API int qi_pack_open(const char *path, qi_pack **out) {
    if (!path || !out) return QI_PACK_EINVAL;
    *out = nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return QI_PACK_EIO;
    uint8_t h[kHeaderBytes];
    struct stat st;
    if (!read_at(fd, h, kHeaderBytes, 0) || fstat(fd, &st) != 0) {
        close(fd);
        return QI_PACK_EIO;
    }
    if (std::memcmp(h, "QIPACK1\0", 8) != 0 || load_le<uint32_t>(h + 12) != kHeaderBytes) {
        close(fd);
        return QI_PACK_EFORMAT;
    }
    qi_pack *p = new (std::nothrow) qi_pack;
    if (!p) {
        close(fd);
        return QI_PACK_EIO;
    }
    p->fd = fd;
    p->tensor_count = load_le<uint32_t>(h + 16);
    p->directory_offset = load_le<uint64_t>(h + 24);
    p->data_offset = load_le<uint64_t>(h + 32);
    p->file_bytes = load_le<uint64_t>(h + 40);
    p->payload_checksum = load_le<uint64_t>(h + 48);
    std::memcpy(p->policy, h + 136, 32);
    p->metadata_offset = load_le<uint64_t>(h + 168);
    p->metadata_bytes = load_le<uint32_t>(h + 176);
    p->metadata_checksum = load_le<uint64_t>(h + 184);
    const uint64_t dir_bytes = static_cast<uint64_t>(p->tensor_count) * kRecordBytes;
    if (p->file_bytes != static_cast<uint64_t>(st.st_size) || p->directory_offset < kHeaderBytes ||
        p->directory_offset + dir_bytes > p->data_offset || p->data_offset > p->file_bytes) {
        qi_pack_close(p);
        return QI_PACK_EFORMAT;
    }
    std::vector<uint8_t> dir(dir_bytes);
    if (!read_at(fd, dir.data(), dir_bytes, p->directory_offset)) {
        qi_pack_close(p);
        return QI_PACK_EIO;
    }
    p->records.resize(p->tensor_count);
    for (uint32_t i = 0; i < p->tensor_count; ++i) {
        const uint8_t *r = dir.data() + static_cast<size_t>(i) * kRecordBytes;
        qi_pack_record &rec = p->records[i];
        std::memcpy(rec.name, r, 128);
        rec.name[128] = 0;
        rec.scheme = load_le<uint32_t>(r + 128);
        rec.rank = load_le<uint32_t>(r + 132);
        for (int d = 0; d < 4; ++d) rec.dims[d] = load_le<uint64_t>(r + 136 + 8 * d);
        rec.group_axis = load_le<uint32_t>(r + 168);
        rec.group_size = load_le<uint32_t>(r + 172);
        rec.scale_type = load_le<uint32_t>(r + 176);
        rec.zero_type = load_le<uint32_t>(r + 180);
        rec.weights_offset = load_le<uint64_t>(r + 184);
        rec.weights_length = load_le<uint64_t>(r + 192);
        rec.scales_offset = load_le<uint64_t>(r + 200);
        rec.scales_length = load_le<uint64_t>(r + 208);
        rec.zeros_offset = load_le<uint64_t>(r + 216);
        rec.zeros_length = load_le<uint64_t>(r + 224);
        rec.elements = load_le<uint64_t>(r + 232);
        rec.tensor_checksum = load_le<uint64_t>(r + 240);
    }
    *out = p;
    return QI_PACK_OK;
}

QI_PACK_API void qi_pack_close(qi_pack *pack) {
    if (!pack) return;
    if (pack->fd >= 0) close(pack->fd);
    delete pack;
}

QI_PACK_API int qi_pack_info(const qi_pack *pack, uint32_t *tensor_count, char *policy33, uint64_t *data_offset,
                             uint64_t *file_bytes) {
    if (!pack) return QI_PACK_EINVAL;
    if (tensor_count) *tensor_count = pack->tensor_count;
    if (policy33) std::memcpy(policy33, pack->policy, 33);
    if (data_offset) *data_offset = pack->data_offset;
    if (file_bytes) *file_bytes = pack->file_bytes;
    return QI_PACK_OK;
}

QI_PACK_API int qi_pack_record_at(const qi_pack *pack, uint32_t index, qi_pack_record *out) {
    if (!pack || !out || index >= pack->tensor_count) return QI_PACK_EINVAL;
    *out = pack->records[index];
    return QI_PACK_OK;
}

QI_PACK_API int qi_pack_find(const qi_pack *pack, const char *name) {
    if (!pack || !name) return -1;
    for (uint32_t i = 0; i < pack->tensor_count; ++i)
        if (!std::strncmp(pack->records[i].name, name, 128)) return static_cast<int>(i);
    return -1;
}

QI_PACK_API int qi_pack_read(const qi_pack *pack, uint64_t offset, uint64_t length, void *dst) {
    if (!pack || (!dst && length) || offset > pack->file_bytes || length > pack->file_bytes - offset)
        return QI_PACK_EINVAL;
    return read_at(pack->fd, dst, length, offset) ? QI_PACK_OK : QI_PACK_EIO;
}

QI_PACK_API int qi_pack_verify(const qi_pack *pack, int expect_transformer) {
    if (!pack) return QI_PACK_EINVAL;
    const int quantized = scheme_of_policy(pack->policy);
    if (quantized < 0) return QI_PACK_EFORMAT;
    // The transformer inventory the reference loads: 297 tensors, 224 of
    // them INT4 block matrices (transformer.cplus:356-357, int4_pack.cplus:831).
    if (expect_transformer && pack->tensor_count != 297) return QI_PACK_EFORMAT;
    const uint64_t directory_end = pack->directory_offset + static_cast<uint64_t>(pack->tensor_count) * kRecordBytes;
    if (pack->metadata_offset < directory_end ||
        pack->metadata_offset + pack->metadata_bytes > pack->data_offset)
        return QI_PACK_ELAYOUT;
    std::vector<uint8_t> chunk(8u << 20);
    uint64_t h = kFnvOffset;
    if (!hash_range(pack->fd, pack->metadata_offset, pack->metadata_bytes, h, chunk)) return QI_PACK_EIO;
    if (h != pack->metadata_checksum) return QI_PACK_EMETADATA;

    uint64_t cursor = pack->data_offset;
    uint32_t matrices = 0;
    for (uint32_t i = 0; i < pack->tensor_count; ++i) {
        const qi_pack_record &r = pack->records[i];
        if (r.scheme == static_cast<uint32_t>(quantized)) {
            ++matrices;
            const uint64_t outputs = r.dims[0], inputs = r.dims[1], group = r.group_size;
            const uint64_t groups = group ? outputs * (inputs / group) : 0;
            if (!group || inputs % group || r.weights_length != outputs * inputs / 2 || r.scales_length != groups * 2 ||
                r.zeros_length != (quantized == static_cast<int>(kSchemeW4A16) ? groups * 2 : 0))
                return QI_PACK_ELAYOUT;
        } else if (r.scheme != kSchemeBf16 && r.scheme != kSchemeFp16) {
            return QI_PACK_ELAYOUT;
        }
        const uint64_t parts[3][2] = {{r.weights_offset, r.weights_length},
                                      {r.scales_offset, r.scales_length},
                                      {r.zeros_offset, r.zeros_length}};
        uint64_t th = kFnvOffset;
        for (const auto &part : parts) {
            if (!part[1]) continue;
            if (part[0] % kAlign || part[0] < cursor || part[0] > pack->file_bytes ||
                part[1] > pack->file_bytes - part[0])
                return QI_PACK_ELAYOUT;
            if (!hash_range(pack->fd, part[0], part[1], th, chunk)) return QI_PACK_EIO;
            cursor = part[0] + part[1];
        }
        if (th != r.tensor_checksum) return QI_PACK_ETENSOR;
    }
    if ((expect_transformer && matrices != 224) || (cursor + kAlign - 1) / kAlign * kAlign != pack->file_bytes)
        return QI_PACK_ELAYOUT;
    uint64_t payload = kFnvOffset;
    if (!hash_range(pack->fd, pack->data_offset, pack->file_bytes - pack->data_offset, payload, chunk))
        return QI_PACK_EIO;
    return payload == pack->payload_checksum ? QI_PACK_OK : QI_PACK_EPAYLOAD;
}
