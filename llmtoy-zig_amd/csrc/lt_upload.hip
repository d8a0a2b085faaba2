// lt_upload.hip -- GGUF tensors between host memory and the planar device
// layout (lt_internal.h).  The raw GGUF blocks cross PCIe in chunks staged
// through pinned host buffers, several chunks in flight on their own streams;
// on the device a byte-shuffle kernel splits each chunk's blocks into the
// planes in HBM (and joins them back for read-back).  The host does one
// memcpy per byte into pinned memory and nothing else.
#include "llmtoy_hip.h"
#include "lt_internal.h"

#include <string.h>

#include <algorithm>
#include <atomic>
#include <thread>
#include <vector>

namespace lt {

namespace {

constexpr int kBlkPerWG = 64;        // blocks per workgroup; chunk starts are multiples of it
constexpr uint32_t kMaxBlockBytes = 210;
constexpr size_t kPad = 16;          // device chunk buffers hold this many bytes past the data

// Plane s of a block type: bytes [off, off + len) of every block, stored
// contiguously per block in plane s (set_planes order: p0, p1, p2, p3).
// Every len is a multiple of 2 and every plane starts 4-byte aligned.
struct PlaneArgs {
    uint8_t *plane[4];
    uint32_t off[4], len[4];
    int nseg;
    uint32_t bb;  // block bytes
};

bool plane_args(const DevTensor &t, PlaneArgs &a) {
    const size_t nblk = t.total_rows * t.blocks_per_row;
    switch (t.type) {
    case LT_TYPE_Q8_0:  // qs (bytes 2..33), d (bytes 0..1)
        a = {{}, {2, 0}, {32, 2}, 2, 34};
        break;
    case LT_TYPE_Q4_K:  // d, dmin, scales (0..15), quants (16..143)
        a = {{}, {0, 16}, {16, 128}, 2, 144};
        break;
    case LT_TYPE_Q6_K:  // ql, qh, scales, d
        a = {{}, {0, 128, 192, 208}, {128, 64, 16, 2}, 4, 210};
        break;
    case LT_TYPE_Q5_0:  // qs (6..21), qh (2..5), d (0..1)
        a = {{}, {6, 2, 0}, {16, 4, 2}, 3, 22};
        break;
    case LT_TYPE_Q5_1:  // qs (8..23), qh (4..7), d and m (0..3)
        a = {{}, {8, 4, 0}, {16, 4, 4}, 3, 24};
        break;
    case LT_TYPE_IQ4_NL:  // qs (2..17), d (0..1)
        a = {{}, {2, 0}, {16, 2}, 2, 18};
        break;
    case LT_TYPE_Q3_K:  // qs (32..95), hmask (0..31), scales (96..107), d (108..109)
        a = {{}, {32, 0, 96, 108}, {64, 32, 12, 2}, 4, 110};
        break;
    default: return false;
    }
    size_t at = 0;
    for (int s = 0; s < a.nseg; s++) {
        a.plane[s] = t.base + at;
        at += nblk * a.len[s];
    }
    return at == t.bytes;
}

// raw: nblk GGUF blocks of this chunk (blocks blk0 .. blk0 + nblk - 1 of the
// tensor), readable up to 3 bytes past nblk * bb.  Each workgroup stages
// kBlkPerWG blocks in LDS with dword loads, then writes each plane's run of
// those blocks as dwords (bytes at a region's ragged end).
__global__ __launch_bounds__(256) void k_blocks_to_planes(const uint8_t *__restrict__ raw, size_t nblk, size_t blk0,
                                                          PlaneArgs a) {
    __shared__ uint32_t lds[(kBlkPerWG * kMaxBlockBytes + 3) / 4];
    const size_t b0 = (size_t)blockIdx.x * kBlkPerWG;
    const uint32_t n = nblk - b0 < (size_t)kBlkPerWG ? (uint32_t)(nblk - b0) : (uint32_t)kBlkPerWG;
    const uint32_t nw = (n * a.bb + 3) / 4;
    const uint32_t *src = reinterpret_cast<const uint32_t *>(raw + b0 * a.bb);
    for (uint32_t w = threadIdx.x; w < nw; w += blockDim.x) lds[w] = src[w];
    __syncthreads();
    const uint8_t *lb = reinterpret_cast<const uint8_t *>(lds);
    for (int s = 0; s < a.nseg; s++) {
        const uint32_t len = a.len[s], off = a.off[s], rb = n * len;
        uint8_t *dst = a.plane[s] + (blk0 + b0) * len;
        for (uint32_t j0 = 4 * threadIdx.x; j0 < rb; j0 += 4 * blockDim.x) {
            if (j0 + 4 <= rb) {
                uint32_t v = 0;
#pragma unroll
                for (uint32_t q = 0; q < 4; q++) {
                    const uint32_t j = j0 + q;
                    v |= (uint32_t)lb[(j / len) * a.bb + off + j % len] << (8 * q);
                }
                *reinterpret_cast<uint32_t *>(dst + j0) = v;
            } else {
                for (uint32_t j = j0; j < rb; j++) dst[j] = lb[(j / len) * a.bb + off + j % len];
            }
        }
    }
}

// Inverse: planes of blocks blk0 .. blk0 + nblk - 1 -> GGUF blocks in raw,
// which must be writable up to 3 bytes past nblk * bb.
__global__ __launch_bounds__(256) void k_planes_to_blocks(uint8_t *__restrict__ raw, size_t nblk, size_t blk0,
                                                          PlaneArgs a) {
    __shared__ uint32_t lds[(kBlkPerWG * kMaxBlockBytes + 3) / 4];
    const size_t b0 = (size_t)blockIdx.x * kBlkPerWG;
    const uint32_t n = nblk - b0 < (size_t)kBlkPerWG ? (uint32_t)(nblk - b0) : (uint32_t)kBlkPerWG;
    const uint32_t nw = (n * a.bb + 3) / 4;
    uint8_t *lb = reinterpret_cast<uint8_t *>(lds);
    for (int s = 0; s < a.nseg; s++) {
        const uint32_t len = a.len[s], off = a.off[s], rb = n * len;
        const uint8_t *src = a.plane[s] + (blk0 + b0) * len;
        for (uint32_t j0 = 4 * threadIdx.x; j0 < rb; j0 += 4 * blockDim.x) {
            if (j0 + 4 <= rb) {
                const uint32_t v = *reinterpret_cast<const uint32_t *>(src + j0);
#pragma unroll
                for (uint32_t q = 0; q < 4; q++) {
                    const uint32_t j = j0 + q;
                    lb[(j / len) * a.bb + off + j % len] = (uint8_t)(v >> (8 * q));
                }
            } else {
                for (uint32_t j = j0; j < rb; j++) lb[(j / len) * a.bb + off + j % len] = src[j];
            }
        }
    }
    __syncthreads();
    uint32_t *dst = reinterpret_cast<uint32_t *>(raw + b0 * a.bb);
    for (uint32_t w = threadIdx.x; w < nw; w += blockDim.x) dst[w] = lds[w];
}

// Streams and staging slots for workers [S.workers, W), kept until the context ends.
hipError_t ensure_staging(UploadStaging &S, int W) {
    hipError_t e = hipSuccess;
    for (; S.workers < W && e == hipSuccess; S.workers++) {
        const int w = S.workers;
        e = hipStreamCreateWithFlags(&S.st[w], hipStreamNonBlocking);
        for (int i = 2 * w; i < 2 * w + 2 && e == hipSuccess; i++) {
            e = hipHostMalloc((void **)&S.pinned[i], kUpChunk, hipHostMallocDefault);
            if (e == hipSuccess) e = hipMalloc((void **)&S.dev[i], kUpChunk + kPad);
            if (e == hipSuccess) e = hipEventCreateWithFlags(&S.ev[i], hipEventDisableTiming);
        }
        if (e != hipSuccess) break;  // this worker's partial resources are freed with the rest
    }
    if (e != hipSuccess) free_staging(S);
    return e;
}

// Blocks per chunk: a multiple of kBlkPerWG whose bytes fit a staging slot.
size_t chunk_blocks(uint32_t bb) { return kUpChunk / bb / kBlkPerWG * kBlkPerWG; }

}  // namespace

void free_staging(UploadStaging &S) {
    for (int w = 0; w < kUpWorkers; w++)
        if (S.st[w]) (void)hipStreamDestroy(S.st[w]), S.st[w] = nullptr;
    for (int i = 0; i < kUpSlots; i++) {
        if (S.pinned[i]) (void)hipHostFree(S.pinned[i]), S.pinned[i] = nullptr;
        if (S.dev[i]) (void)hipFree(S.dev[i]), S.dev[i] = nullptr;
        if (S.ev[i]) (void)hipEventDestroy(S.ev[i]), S.ev[i] = nullptr;
    }
    S.workers = 0;
}

hipError_t upload_planar(UploadStaging &S, int device, const DevTensor &t, const uint8_t *src) {
    PlaneArgs pa{};
    const bool f32 = t.type == LT_TYPE_F32;
    if (!f32 && !plane_args(t, pa)) return hipErrorInvalidValue;
    const uint32_t bb = f32 ? 4u : pa.bb;
    const size_t nblk = t.bytes / bb, CH = chunk_blocks(bb);
    if (nblk * bb != t.bytes || CH == 0) return hipErrorInvalidValue;
    const size_t nchunks = (nblk + CH - 1) / CH;
    const int W = (int)std::min<size_t>(kUpWorkers, nchunks);
    hipError_t e = ensure_staging(S, W);
    if (e != hipSuccess) return e;
    std::atomic<int> err{(int)hipSuccess};

    // worker w moves chunks w, w + W, ... through its two slots on its own stream
    auto work = [&](int w, bool own_thread) {
        hipError_t e = own_thread ? hipSetDevice(device) : hipSuccess;
        int use = 0;
        for (size_t c = (size_t)w; c < nchunks && e == hipSuccess && err.load() == (int)hipSuccess;
             c += (size_t)W, use++) {
            const int slot = 2 * w + (use & 1);
            if (use >= 2) e = hipEventSynchronize(S.ev[slot]);  // the slot's previous chunk is done
            if (e != hipSuccess) break;
            const size_t first = c * CH, nb = std::min(CH, nblk - first);
            memcpy(S.pinned[slot], src + first * bb, nb * bb);
            if (f32) {
                e = hipMemcpyAsync(t.base + first * bb, S.pinned[slot], nb * bb, hipMemcpyHostToDevice, S.st[w]);
            } else {
                e = hipMemcpyAsync(S.dev[slot], S.pinned[slot], nb * bb, hipMemcpyHostToDevice, S.st[w]);
                if (e == hipSuccess) {
                    k_blocks_to_planes<<<(unsigned)((nb + kBlkPerWG - 1) / kBlkPerWG), 256, 0, S.st[w]>>>(
                        S.dev[slot], nb, first, pa);
                    e = hipGetLastError();
                }
            }
            if (e == hipSuccess) e = hipEventRecord(S.ev[slot], S.st[w]);
        }
        const hipError_t e2 = hipStreamSynchronize(S.st[w]);
        if (e == hipSuccess) e = e2;
        if (e != hipSuccess) {
            int expect = (int)hipSuccess;
            err.compare_exchange_strong(expect, (int)e);
        }
    };
    if (W == 1) {
        work(0, false);
    } else {
        std::vector<std::thread> th;
        th.reserve(W);
        for (int w = 0; w < W; w++) th.emplace_back(work, w, true);
        for (auto &x : th) x.join();
    }
    return (hipError_t)err.load();
}

hipError_t download_planar(UploadStaging &S, const DevTensor &t, uint8_t *dst) {
    PlaneArgs pa{};
    const bool f32 = t.type == LT_TYPE_F32;
    if (!f32 && !plane_args(t, pa)) return hipErrorInvalidValue;
    const uint32_t bb = f32 ? 4u : pa.bb;
    const size_t nblk = t.bytes / bb, CH = chunk_blocks(bb);
    if (nblk * bb != t.bytes || CH == 0) return hipErrorInvalidValue;
    hipError_t e = ensure_staging(S, 1);
    for (size_t first = 0; first < nblk && e == hipSuccess; first += CH) {
        const size_t nb = std::min(CH, nblk - first);
        if (f32) {
            e = hipMemcpyAsync(S.pinned[0], t.base + first * bb, nb * bb, hipMemcpyDeviceToHost, S.st[0]);
        } else {
            k_planes_to_blocks<<<(unsigned)((nb + kBlkPerWG - 1) / kBlkPerWG), 256, 0, S.st[0]>>>(S.dev[0], nb,
                                                                                               first, pa);
            e = hipGetLastError();
            if (e == hipSuccess)
                e = hipMemcpyAsync(S.pinned[0], S.dev[0], nb * bb, hipMemcpyDeviceToHost, S.st[0]);
        }
        if (e == hipSuccess) e = hipStreamSynchronize(S.st[0]);
        if (e == hipSuccess) memcpy(dst + first * bb, S.pinned[0], nb * bb);
    }
    return e;
}

}  // namespace lt
