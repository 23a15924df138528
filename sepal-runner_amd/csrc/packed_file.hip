// Packed-weight files: the int8 weights and float32 scales of one matrix, as the packer left them, with the identity
// of what they were packed from, so that a later load can skip the packer (runner/cuda/src/cuda_engine.cpp:545-627
// re-quantizes at every load; the file is the cache of that work).
//
// Layout (little-endian, 64-byte header, then the payload):
//    0  8  magic "SPW8G128"
//    8  4  format version (1)
//   12  4  quantizer rule (SEPAL_HIP_RULE_DIVIDE / _RECIPROCAL)
//   16  4  row layout (0 plain rows, 1 the 64-row gate/up interleave)
//   20  4  zero
//   24  8  rows
//   32  8  k
//   40  8  fingerprint of the source weights the caller packed (sepal_hip_weight_fingerprint of their bytes)
//   48  8  fingerprint of the int8 payload
//   56  8  fingerprint of the scale payload
//   64     rows x k int8 (row stride k), then rows x k / 128 float32 (row stride k / 128)
//
// The fingerprint is a 64-bit hash of a byte range computed on the device: 8-byte words (the tail zero-padded), word i
// folded into lane i mod 65536 with the splitmix64 finalizer (Steele, Lea and Flood, "Fast splittable pseudorandom
// number generators", OOPSLA 2014) over (word + golden-ratio increments), the 65536 lane values then folded in order by
// 256 threads of 256 values each and by one thread over those, and the byte count folded last. The grid is fixed, so
// the value does not depend on the device. (The reference fingerprints device memory the same way in spirit, with its
// own mixing: runner/cuda/src/engine_kernels.cu:26-54.)
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>

#include "common.hpp"
#include "gemm_kernels.hpp"

namespace sepal::hip {
namespace packfile {

constexpr int kLanes = 65536, kThreads = 256;
constexpr unsigned long long kGolden = 0x9E3779B97F4A7C15ull;

__device__ __forceinline__ unsigned long long mix64(unsigned long long z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ void __launch_bounds__(kThreads) lane_kernel(const unsigned char* __restrict__ data, std::size_t bytes,
                                                        unsigned long long* __restrict__ lanes) {
    const std::size_t lane = static_cast<std::size_t>(blockIdx.x) * kThreads + threadIdx.x;
    const std::size_t words = (bytes + 7) / 8, full = bytes / 8;
    const auto* w64 = reinterpret_cast<const unsigned long long*>(data);
    unsigned long long h = mix64(lane + 1);
    // the lane's whole words eight at a time, all eight loads in flight before the chain folds them in order
    constexpr int B = 8;
    std::size_t i = lane;
    for (; i + (B - 1) * static_cast<std::size_t>(kLanes) < full; i += B * static_cast<std::size_t>(kLanes)) {
        unsigned long long w[B];
#pragma unroll
        for (int j = 0; j < B; ++j) w[j] = w64[i + j * static_cast<std::size_t>(kLanes)];
#pragma unroll
        for (int j = 0; j < B; ++j) h = mix64(h ^ (w[j] + kGolden * (i + j * static_cast<std::size_t>(kLanes) + 1)));
    }
    for (; i < words; i += kLanes) {
        unsigned long long w = 0;
        if (i < full) {
            w = w64[i];
        } else {
            for (std::size_t b = 8 * i; b < bytes; ++b) w |= static_cast<unsigned long long>(data[b]) << (8 * (b - 8 * i));
        }
        h = mix64(h ^ (w + kGolden * (i + 1)));
    }
    lanes[lane] = h;
}

// 256 threads fold 256 lanes each in order, then thread 0 folds the 256 results in order and the byte count
__global__ void __launch_bounds__(kThreads) fold_kernel(const unsigned long long* __restrict__ lanes, std::size_t bytes,
                                                        unsigned long long* __restrict__ out) {
    __shared__ unsigned long long part[kThreads];
    unsigned long long h = 0;
    for (int j = 0; j < kLanes / kThreads; ++j) h = mix64(h ^ lanes[threadIdx.x * (kLanes / kThreads) + j]);
    part[threadIdx.x] = h;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long r = 0;
        for (int t = 0; t < kThreads; ++t) r = mix64(r ^ part[t]);
        out[0] = mix64(r ^ static_cast<unsigned long long>(bytes));
    }
}

struct Header {
    char magic[8];
    std::uint32_t version, rule, layout, zero;
    std::uint64_t rows, k, source_fp, q_fp, s_fp;
};
static_assert(sizeof(Header) == 64, "64-byte header");
constexpr char kMagic[8] = {'S', 'P', 'W', '8', 'G', '1', '2', '8'};

struct FileCloser {
    void operator()(std::FILE* f) const { std::fclose(f); }
};
struct HostFree {
    void operator()(void* p) const { (void)hipHostFree(p); }
};

constexpr std::size_t kStage = std::size_t{32} << 20;  // pinned staging chunk

std::unique_ptr<unsigned char, HostFree> pinned(std::size_t bytes) {
    void* p = nullptr;
    if (hipHostMalloc(&p, bytes, hipHostMallocDefault) != hipSuccess) throw std::bad_alloc();
    return std::unique_ptr<unsigned char, HostFree>(static_cast<unsigned char*>(p));
}

void sync(hipStream_t stream, const char* what) {
    const hipError_t e = hipStreamSynchronize(stream);
    if (e != hipSuccess) throw LaunchError(std::string(what) + ": " + hipGetErrorString(e));
}

// Copies `rows` rows of `row_bytes` (device row stride `ld_bytes`) to the file, through the pinned chunk.
void write_rows(std::FILE* f, const unsigned char* dev, std::size_t ld_bytes, std::size_t rows, std::size_t row_bytes,
                unsigned char* stage, hipStream_t stream) {
    const std::size_t per = kStage / row_bytes;
    for (std::size_t r0 = 0; r0 < rows; r0 += per) {
        const std::size_t n = rows - r0 < per ? rows - r0 : per;
        if (hipMemcpy2DAsync(stage, row_bytes, dev + r0 * ld_bytes, ld_bytes, row_bytes, n, hipMemcpyDeviceToHost, stream) != hipSuccess)
            throw LaunchError("packed file: device to host copy failed");
        sync(stream, "packed file: device to host copy");
        if (std::fwrite(stage, 1, n * row_bytes, f) != n * row_bytes) throw IoError("packed file: write failed");
    }
}

void read_rows(std::FILE* f, unsigned char* dev, std::size_t ld_bytes, std::size_t rows, std::size_t row_bytes,
               unsigned char* stage, hipStream_t stream) {
    const std::size_t per = kStage / row_bytes;
    for (std::size_t r0 = 0; r0 < rows; r0 += per) {
        const std::size_t n = rows - r0 < per ? rows - r0 : per;
        if (std::fread(stage, 1, n * row_bytes, f) != n * row_bytes) throw IoError("packed file: truncated payload");
        if (hipMemcpy2DAsync(dev + r0 * ld_bytes, ld_bytes, stage, row_bytes, row_bytes, n, hipMemcpyHostToDevice, stream) != hipSuccess)
            throw LaunchError("packed file: host to device copy failed");
        sync(stream, "packed file: host to device copy");  // the chunk is reused
    }
}

} // namespace packfile

void launch_fingerprint(const void* data, std::size_t bytes, std::uint64_t* out, void* lanes, hipStream_t stream) {
    packfile::lane_kernel<<<dim3(packfile::kLanes / packfile::kThreads), dim3(packfile::kThreads), 0, stream>>>(
        static_cast<const unsigned char*>(data), bytes, static_cast<unsigned long long*>(lanes));
    check_launch("fingerprint lane kernel launch");
    packfile::fold_kernel<<<dim3(1), dim3(packfile::kThreads), 0, stream>>>(static_cast<const unsigned long long*>(lanes), bytes,
                                                                        reinterpret_cast<unsigned long long*>(out));
    check_launch("fingerprint fold kernel launch");
}

std::size_t fingerprint_scratch_bytes() { return static_cast<std::size_t>(packfile::kLanes) * 8 + 256; }

// The fingerprint of a device range, returned to the host (synchronous). `scratch` holds fingerprint_scratch_bytes().
static std::uint64_t fingerprint_now(const void* data, std::size_t bytes, void* scratch, hipStream_t stream) {
    auto* lanes = static_cast<unsigned char*>(scratch);
    auto* out = reinterpret_cast<std::uint64_t*>(lanes + static_cast<std::size_t>(packfile::kLanes) * 8);
    launch_fingerprint(data, bytes, out, lanes, stream);
    std::uint64_t h = 0;
    if (hipMemcpyAsync(&h, out, 8, hipMemcpyDeviceToHost, stream) != hipSuccess) throw LaunchError("fingerprint copy failed");
    packfile::sync(stream, "fingerprint");
    return h;
}

void packed_save(const char* path, const std::int8_t* q, std::size_t ld_q, const float* s, std::size_t ld_s,
                 std::size_t rows, std::size_t k, int rule, int layout, std::uint64_t source_fp, void* scratch,
                 hipStream_t stream) {
    using namespace packfile;
    // fingerprints of the payload as it will sit in the file (contiguous rows): hash a contiguous copy when strided
    Header h{};
    std::memcpy(h.magic, kMagic, 8);
    h.version = 1;
    h.rule = static_cast<std::uint32_t>(rule);
    h.layout = static_cast<std::uint32_t>(layout);
    h.rows = rows;
    h.k = k;
    h.source_fp = source_fp;
    if (ld_q != k || ld_s != k / 128) throw InvalidArgument("packed_save: q and s must be contiguous (ld_q = k, ld_s = k / 128)");
    h.q_fp = fingerprint_now(q, rows * k, scratch, stream);
    h.s_fp = fingerprint_now(s, rows * (k / 128) * sizeof(float), scratch, stream);
    std::unique_ptr<std::FILE, FileCloser> f(std::fopen(path, "wb"));
    if (!f) throw IoError(std::string("packed_save: cannot open ") + path);
    if (std::fwrite(&h, sizeof h, 1, f.get()) != 1) throw IoError("packed_save: header write failed");
    auto stage = pinned(kStage);
    write_rows(f.get(), reinterpret_cast<const unsigned char*>(q), k, rows, k, stage.get(), stream);
    write_rows(f.get(), reinterpret_cast<const unsigned char*>(s), k / 128 * sizeof(float), rows, k / 128 * sizeof(float),
               stage.get(), stream);
    if (std::fflush(f.get()) != 0) throw IoError("packed_save: flush failed");
}

void packed_load(const char* path, std::int8_t* q, std::size_t ld_q, float* s, std::size_t ld_s, std::size_t rows,
                 std::size_t k, int rule, int layout, std::uint64_t source_fp, void* scratch, hipStream_t stream) {
    using namespace packfile;
    if (ld_q != k || ld_s != k / 128) throw InvalidArgument("packed_load: q and s must be contiguous (ld_q = k, ld_s = k / 128)");
    std::unique_ptr<std::FILE, FileCloser> f(std::fopen(path, "rb"));
    if (!f) throw IoError(std::string("packed_load: cannot open ") + path);
    Header h{};
    if (std::fread(&h, sizeof h, 1, f.get()) != 1 || std::memcmp(h.magic, kMagic, 8) != 0 || h.version != 1 || h.zero != 0)
        throw IoError("packed_load: not a packed-weight file of format 1");
    if (h.rows != rows || h.k != k || h.rule != static_cast<std::uint32_t>(rule) || h.layout != static_cast<std::uint32_t>(layout) ||
        h.source_fp != source_fp)
        throw StaleError("packed_load: the file holds other weights (shape, rule, layout or source fingerprint differ)");
    auto stage = pinned(kStage);
    read_rows(f.get(), reinterpret_cast<unsigned char*>(q), k, rows, k, stage.get(), stream);
    read_rows(f.get(), reinterpret_cast<unsigned char*>(s), k / 128 * sizeof(float), rows, k / 128 * sizeof(float), stage.get(),
              stream);
    if (fingerprint_now(q, rows * k, scratch, stream) != h.q_fp || fingerprint_now(s, rows * (k / 128) * sizeof(float), scratch, stream) != h.s_fp)
        throw IoError("packed_load: the payload does not match its fingerprints (corrupt file)");
}

} // namespace sepal::hip
