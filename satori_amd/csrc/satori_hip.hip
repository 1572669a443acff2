// Host runtime of libsatori_hip.so: contexts, resident matrices, launches, and the C ABI declared in
// include/satori_hip.h. Every entry point converts internal failures into a status code plus a per-thread
// message, and host-buffer MatVec calls copy into the caller's output only after the stream has
// completed without error (IQuantizedMatrix contract, src/Satori.Core/IQuantizedMatrix.cs:6).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/satori_hip.h"
#include "gguf.hpp"
#include "host_shapes.hpp"
#include "kernels.hpp"

namespace satori {
namespace {

thread_local std::string g_last_error;

}  // namespace

void record_error(const std::string& message) { g_last_error = message; }

namespace {

// Slack after every payload: the misaligned-block loaders read up to 4 bytes past a block.
constexpr size_t kPayloadSlack = 256;

// The ABI's format codes are the kernels' own (shapes carry the ABI code into the launches).
static_assert(SATORI_HIP_Q8_0 == satori::kQ8_0 && SATORI_HIP_Q4_0 == satori::kQ4_0 && SATORI_HIP_Q4_K == satori::kQ4_K &&
                  SATORI_HIP_Q6_K == satori::kQ6_K && SATORI_HIP_TERNARY2 == satori::kTernary2,
              "format codes");

void check_hip(hipError_t e, const char* what) {
    if (e != hipSuccess)
        fail(e == hipErrorOutOfMemory ? SATORI_HIP_E_OUT_OF_MEMORY : SATORI_HIP_E_DEVICE,
             std::string(what) + ": " + hipGetErrorString(e));
}

// Device buffer that only grows.
struct DeviceBuffer {
    void* ptr = nullptr;
    size_t bytes = 0;
    void reserve(size_t need) {
        if (need <= bytes) return;
        if (ptr) (void)hipFree(ptr);
        ptr = nullptr;
        bytes = 0;
        check_hip(hipMalloc(&ptr, need), "hipMalloc");
        bytes = need;
    }
    void release() {
        if (ptr) (void)hipFree(ptr);
        ptr = nullptr;
        bytes = 0;
    }
};

struct PinnedBuffer {
    void* ptr = nullptr;
    size_t bytes = 0;
    void reserve(size_t need) {
        if (need <= bytes) return;
        if (ptr) (void)hipHostFree(ptr);
        ptr = nullptr;
        bytes = 0;
        check_hip(hipHostMalloc(&ptr, need, hipHostMallocDefault), "hipHostMalloc");
        bytes = need;
    }
    void release() {
        if (ptr) (void)hipHostFree(ptr);
        ptr = nullptr;
        bytes = 0;
    }
};

}  // namespace
}  // namespace satori

struct satori_hip_context {
    int device = 0;
    hipStream_t stream = nullptr;
    std::mutex lock;
    bool live = true;
    int matrices = 0;
    satori::DeviceBuffer x, y, q8k;
    satori::DeviceBuffer upload_stage, upload_flag;  // packed payloads on their way into the device layouts
    // Split-attention partials (grouped attention over long prefixes), one buffer per stream the attention
    // runs on, so attentions on different streams never share one; attentions on one stream run in order.
    std::vector<std::pair<hipStream_t, satori::DeviceBuffer>> attention;
    int attention_steps = 0;         // live captured steps whose graph uses the context stream's buffer
    bool captured_attention = false; // the capture in progress enqueued a split attention
    // The device address of the no-allocation attention's partials on this context's device (the file-scope
    // array of transformer_ops.hip), resolved once when the context is created.
    double* static_attention = nullptr;
    satori::PinnedBuffer host_x, host_y;
    // Stream capture (satori_hip_capture_begin / _end): the matrices and groups launched on the context
    // stream while capturing, referenced by the step the capture becomes.
    bool capturing = false;
    std::vector<satori_hip_matrix*> captured_matrices;
    std::vector<satori_hip_group*> captured_groups;
};

struct satori_hip_matrix {
    satori_hip_context* context = nullptr;
    satori::Shape shape;
    uint8_t* payload = nullptr;  // device: the packed payload, or the panel layout for Ternary2
    int64_t device_bytes = 0;    // bytes at `payload` (slack excluded)
    satori::T2Plan plan{};       // Ternary2 launch plan of a single execution
    void* scratch = nullptr;     // Ternary2 range scratch (device), when the plan has several ranges
    uint32_t t2_generation = 0;  // the last Ternary2 launch's tag in the scratch's exchange slots
    satori::DeviceBuffer q8k;    // activations of the last many-position product (K formats: packed Q8_K;
                                 // Q8_0 / Q4_0: split bf16 parts)
    satori::DeviceBuffer planes; // Q6_K: the matrix-core weight planes, built by the first many-position product
    int groups = 0;              // live groups and captured steps that launch this matrix
    int steps = 0;               // captured steps that launch this matrix directly (they hold its q8k buffer)
    bool live = true;
};

struct satori_hip_group {
    satori_hip_context* context = nullptr;
    satori::Shape shape;
    int count = 0;
    bool quantized = false;
    int rows_max = 0;
    satori::MatDesc* descriptors = nullptr;   // device
    std::vector<satori::MatDesc> host;         // the same descriptors on the host
    satori::DeviceBuffer batch;                // K groups: packed Q8_K activations of many-position calls
    satori::InputTransform input{};            // K groups: input computed in the launch (kInputPlain: read x)
    satori::OutputSwiGluQ8K output{};          // gate/up K groups: SwiGlu and its Q8_K bytes carried on (or none)
    satori::DeviceBuffer counters;             // the arrival counts of `output` (one per 256 rows)
    satori::DeviceBuffer shared_q8k;           // large K groups sharing one input: its Q8_K bytes, made per launch
    satori::T2Plan plan{};                     // Ternary2 groups
    void* scratch = nullptr;                   // Ternary2 range scratch (device)
    uint32_t t2_generation = 0;                // the last Ternary2 launch's tag in the scratch's exchange slots
    std::vector<satori_hip_matrix*> members;   // distinct member matrices (each counts this group)
    int steps = 0;                             // live steps that replay this group
    bool live = true;
};

struct satori_hip_gguf {
    satori::GgufFile* file = nullptr;  // null once closed (the handle stays as a tombstone)
    bool live = true;
};

struct satori_hip_step {
    satori_hip_context* context = nullptr;
    std::vector<satori_hip_group*> groups;     // in launch order (each counts this step)
    std::vector<satori_hip_matrix*> matrices;  // launched directly in a captured step (each counts it)
    bool attention = false;                    // the graph uses the context's split-attention workspace
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    bool live = true;
};

namespace satori {
namespace {

int succeed() {
    g_last_error.clear();
    return SATORI_HIP_OK;
}

template <class F>
int guarded(F&& body) {
    try {
        body();
        return succeed();
    } catch (const Failure& f) {
        g_last_error = f.message;
        return f.status;
    } catch (const std::bad_alloc&) {
        g_last_error = "Out of host memory.";
        return SATORI_HIP_E_OUT_OF_MEMORY;
    } catch (...) {
        g_last_error = "Unexpected failure.";
        return SATORI_HIP_E_DEVICE;
    }
}

void require(const void* p, const char* name) {
    if (!p) fail(SATORI_HIP_E_ARGUMENT_NULL, std::string("Value cannot be null. (Parameter '") + name + "')");
}

void require_live(const satori_hip_context* c) {
    require(c, "context");
    if (!c->live) fail(SATORI_HIP_E_OBJECT_DISPOSED, "Cannot access a disposed object. Object name: 'satori_hip_context'.");
}

void require_live(const satori_hip_matrix* m) {
    require(m, "matrix");
    if (!m->live || !m->context->live)
        fail(SATORI_HIP_E_OBJECT_DISPOSED, "Cannot access a disposed object. Object name: 'satori_hip_matrix'.");
}

void set_device(const satori_hip_context* c) { check_hip(hipSetDevice(c->device), "hipSetDevice"); }

// Calls that synchronise, allocate or copy through the host cannot be recorded into a graph.
void require_not_capturing(const satori_hip_context* c) {
    if (c->capturing)
        fail(SATORI_HIP_E_INVALID_OPERATION, "Not allowed while the context stream is being captured.");
}

// Work enqueued on the context stream while capturing becomes part of the step: keep what it launches alive.
void note_launch(satori_hip_context* c, satori_hip_matrix* m, hipStream_t stream) {
    if (c->capturing && stream == c->stream) c->captured_matrices.push_back(m);
}

LaunchShape launch_shape(const Shape& s, int positions, int rows_max) {
    LaunchShape l{};
    l.format = s.format == SATORI_HIP_TERNARY2 ? kTernary2 : s.format;
    l.columns = s.columns;
    l.block_size = s.block_size;
    l.blocks = s.blocks;
    l.row_bytes = s.row_bytes;
    l.positions = positions;
    l.rows_max = rows_max;
    return l;
}

bool is_k(const Shape& s) { return s.format == SATORI_HIP_Q4_K || s.format == SATORI_HIP_Q6_K; }

// Enqueue one FP32-activation product: x [positions][C] -> y [positions][R], all device pointers. Q8_0 and
// Q4_0 over fbatch_min_positions() positions or more run on the matrix cores, 256 positions per launch pair,
// with the split activations in the matrix's activation buffer (executions of one matrix that overlap in
// time race on it).
void enqueue_float(satori_hip_matrix* m, const float* x, int positions, float* y, hipStream_t stream) {
    const Shape& s = m->shape;
    if ((s.format == SATORI_HIP_Q8_0 || s.format == SATORI_HIP_Q4_0) && positions >= fbatch_min_positions()) {
        constexpr int kChunk = 256;
        const size_t need = fbatch_workspace_bytes(s.columns, std::min(positions, kChunk));
        if (m->context->capturing && m->q8k.bytes < need)
            fail(SATORI_HIP_E_INVALID_OPERATION,
                 "Run this many-position product once before capturing it (its workspace is allocated on first use).");
        if (m->steps > 0 && m->q8k.bytes < need)  // a captured step holds the current buffer
            fail(SATORI_HIP_E_INVALID_OPERATION,
                 "The workspace of this matrix cannot grow while a captured step launches it: destroy the step, "
                 "or run the largest product before capturing.");
        m->q8k.reserve(need);
        for (int p0 = 0; p0 < positions; p0 += kChunk) {
            const int n = std::min(kChunk, positions - p0);
            check_hip(launch_gemv_fbatch(m->payload, s.format, x + static_cast<int64_t>(p0) * s.columns,
                                         static_cast<uint8_t*>(m->q8k.ptr), y + static_cast<int64_t>(p0) * s.rows,
                                         s.rows, s.columns, n, stream),
                      "matrix-core gemv launch");
        }
        return;
    }
    MatDesc d{m->payload, x, y, s.rows, 0};
    const LaunchShape l = launch_shape(s, positions, s.rows);
    if (s.format == SATORI_HIP_TERNARY2)
        check_hip(launch_t2(d, nullptr, 1, l, m->plan, m->scratch, next_t2_generation(m->t2_generation), stream),
                  "Ternary2 launch");
    else
        check_hip(launch_gemv_float(d, nullptr, 1, l, stream), "gemv launch");
}

// The weights a many-position (matrix-core) product reads: the resident payload for Q4_K; for Q6_K the weight
// planes, built on the device by the matrix's first many-position product (2.02 bytes a weight, kept until
// the matrix is destroyed). The build completes before this returns, so a later product on any stream reads
// whole planes; it cannot be recorded in a capture.
const uint8_t* ensure_planes(satori_hip_matrix* m, hipStream_t stream) {
    if (m->shape.format != SATORI_HIP_Q6_K) return m->payload;
    if (m->planes.ptr) return static_cast<const uint8_t*>(m->planes.ptr);
    if (m->context->capturing)
        fail(SATORI_HIP_E_INVALID_OPERATION,
             "Run this many-position product once before capturing it (its workspace is allocated on first use).");
    const Shape& s = m->shape;
    m->planes.reserve(kmfma_planes_bytes(s.rows, s.blocks));
    hipError_t e = launch_kmfma_planes(m->payload, s.rows, s.blocks, static_cast<uint8_t*>(m->planes.ptr), stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    if (e != hipSuccess) {
        m->planes.release();
        check_hip(e, "weight planes");
    }
    return static_cast<const uint8_t*>(m->planes.ptr);
}

// Enqueue the Q8_K integer product. Few positions: one kernel that quantizes the activations itself; many:
// quantize all positions into the matrix's Q8_K buffer, then the matrix-core product (same outputs). The
// buffer belongs to the matrix, so many-position executions of one matrix that overlap in time race.
void enqueue_kint(satori_hip_matrix* m, const float* x, int positions, float* y, hipStream_t stream) {
    const Shape& s = m->shape;
    if (positions >= kmfma_min_positions()) {
        const size_t need = kmfma_workspace_bytes(s.blocks, positions);
        if (m->context->capturing && m->q8k.bytes < need)
            fail(SATORI_HIP_E_INVALID_OPERATION,
                 "Run this many-position product once before capturing it (its workspace is allocated on first use).");
        if (m->steps > 0 && m->q8k.bytes < need)  // a captured step holds the current buffer
            fail(SATORI_HIP_E_INVALID_OPERATION,
                 "The workspace of this matrix cannot grow while a captured step launches it: destroy the step, "
                 "or run the largest product before capturing.");
        const uint8_t* planes = ensure_planes(m, stream);
        m->q8k.reserve(need);
        check_hip(launch_gemv_kmfma(planes, s.format, x, static_cast<uint8_t*>(m->q8k.ptr), y, s.rows, s.blocks,
                                    s.row_bytes, positions, stream),
                  "matrix-core gemv launch");
        return;
    }
    MatDesc d{m->payload, x, y, s.rows, 0};
    check_hip(launch_gemv_kint(&d, nullptr, 1, launch_shape(s, positions, s.rows), stream), "integer gemv launch");
}

bool overlaps(const void* a, size_t a_bytes, const void* b, size_t b_bytes) {
    const uintptr_t a0 = reinterpret_cast<uintptr_t>(a), b0 = reinterpret_cast<uintptr_t>(b);
    return a0 < b0 + b_bytes && b0 < a0 + a_bytes;
}

// Whether [p, p + bytes) overlaps a buffer that input transform t reads or writes (columns: the group's width).
bool overlaps_transform(const void* p, size_t bytes, const InputTransform& t, int columns) {
    const size_t n = static_cast<size_t>(columns) * sizeof(float);
    switch (t.kind) {
        case kInputAddRmsNorm:
            return overlaps(p, bytes, t.a, n) || (t.b && overlaps(p, bytes, t.b, n)) || overlaps(p, bytes, t.w, n) ||
                   (t.residual_out && overlaps(p, bytes, t.residual_out, n));
        case kInputSwiGlu: return overlaps(p, bytes, t.a, n) || overlaps(p, bytes, t.b, n);
        case kInputQ8K: return overlaps(p, bytes, t.a, static_cast<size_t>(columns / 256) * kQ8KBlockBytes);
        default: return false;
    }
}

// Scratch of a Ternary2 plan, with the plan's tables copied to its start.
void* allocate_t2_scratch(const T2Plan& plan) {
    if (plan.workgroups < 1)
        fail(SATORI_HIP_E_NOT_SUPPORTED, "Ternary2 launch too large: more than 2^31 - 1 tiles of work.");
    void* p = nullptr;
    check_hip(hipMalloc(&p, plan.scratch_bytes), "hipMalloc");
    const hipError_t e = hipMemcpy(p, plan.tables.data(), plan.tables.size(), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(p);
        check_hip(e, "launch table upload");
    }
    return p;
}

// Packed bytes staged on the device per chunk of the regrouping uploads (a chunk holds at least one unit).
constexpr int64_t kUploadStageBytes = 64ll << 20;

// Bytes of the device layout of a matrix of shape s.
int64_t device_layout_bytes(const Shape& s) {
    if (s.format == SATORI_HIP_TERNARY2) return t2_layout(s.rows, s.columns, s.block_size).bytes;
    return s.byte_length;
}

// Copies a packed payload into the device layout at `out` (device_layout_bytes of it, zeroed here): formats
// stored as packed are copied, the others pass through the context's staging buffer in chunks of whole units
// (Ternary2: 64-row panels; Q6_K, Q8_0, Q4_0: blocks) and are regrouped on the device (upload.hip); with
// `bitplanes` a Ternary2-shaped payload holds ternary bitplane blocks, converted on the way. Returns false when
// a Ternary2 block breaks the payload rule (the device check of Ternary2Matrix.ValidatePayload).
bool upload_layout(satori_hip_context* c, const Shape& s, const uint8_t* payload, uint8_t* out, bool bitplanes) {
    const int64_t out_bytes = device_layout_bytes(s);
    const bool t2 = s.format == SATORI_HIP_TERNARY2;
    if (!t2 && s.format != SATORI_HIP_Q6_K && s.format != SATORI_HIP_Q8_0 && s.format != SATORI_HIP_Q4_0) {
        check_hip(hipMemcpy(out, payload, static_cast<size_t>(out_bytes), hipMemcpyHostToDevice), "weight upload");
        return true;
    }
    hipStream_t st = c->stream;
    check_hip(hipMemsetAsync(out, 0, static_cast<size_t>(out_bytes), st), "weight upload");
    const int64_t n = static_cast<int64_t>(s.rows) * s.blocks;
    const int panels = (s.rows + kT2PanelRows - 1) / kT2PanelRows;
    const int64_t unit_bytes = t2 ? kT2PanelRows * s.row_bytes : s.block_bytes;
    const int64_t units = t2 ? panels : n;
    const int64_t per_chunk = std::max<int64_t>(1, kUploadStageBytes / unit_bytes);
    c->upload_stage.reserve(static_cast<size_t>(std::min(per_chunk * unit_bytes, s.byte_length)));
    uint8_t* stage = static_cast<uint8_t*>(c->upload_stage.ptr);
    uint32_t* flag = nullptr;
    if (t2) {
        c->upload_flag.reserve(sizeof(uint32_t));
        flag = static_cast<uint32_t*>(c->upload_flag.ptr);
        check_hip(hipMemsetAsync(flag, 0, sizeof(uint32_t), st), "weight upload");
    }
    const T2Layout l = t2 ? t2_layout(s.rows, s.columns, s.block_size) : T2Layout{};
    for (int64_t u0 = 0; u0 < units; u0 += per_chunk) {
        const int64_t count = std::min(per_chunk, units - u0);
        const uint8_t* src = payload + u0 * unit_bytes;
        if (t2) {
            const int rows = static_cast<int>(std::min<int64_t>(count * kT2PanelRows, s.rows - u0 * kT2PanelRows));
            check_hip(hipMemcpyAsync(stage, src, static_cast<size_t>(rows * s.row_bytes), hipMemcpyHostToDevice, st),
                      "weight upload");
            const T2Regroup r{static_cast<int>(u0), rows, s.columns, s.block_size, s.blocks, s.block_bytes,
                              s.row_bytes, l.chunks, l.slots, l.codes_bytes, bitplanes ? 1 : 0};
            check_hip(launch_t2_regroup(stage, r, out, flag, st), "weight regroup");
        } else {
            check_hip(hipMemcpyAsync(stage, src, static_cast<size_t>(count * unit_bytes), hipMemcpyHostToDevice, st),
                      "weight upload");
            if (s.format == SATORI_HIP_Q6_K)
                check_hip(launch_q6k_regroup(stage, u0, count, n, out, st), "weight regroup");
            else
                check_hip(launch_legacy_regroup(stage, u0, count, n, s.format, out, st), "weight regroup");
        }
    }
    uint32_t bad = 0;
    if (t2) check_hip(hipMemcpyAsync(&bad, flag, sizeof(bad), hipMemcpyDeviceToHost, st), "weight upload");
    check_hip(hipStreamSynchronize(st), "weight upload");
    return bad == 0;
}

// Device allocations of one matrix: the weights (+ slack) and, for a split Ternary2 plan, its scratch.
// Executions of one matrix that overlap in time (device entry points on different streams) share that
// scratch and must be serialised by the caller.
void allocate_matrix(satori_hip_matrix* m, int64_t device_bytes) {
    check_hip(hipMalloc(reinterpret_cast<void**>(&m->payload), static_cast<size_t>(device_bytes) + kPayloadSlack),
              "hipMalloc");
    m->device_bytes = device_bytes;
    if (m->shape.format == SATORI_HIP_TERNARY2) {
        m->plan = t2_plan(m->shape.rows, m->shape.columns, m->shape.block_size, 1, 1);
        m->scratch = allocate_t2_scratch(m->plan);
    }
}

void free_matrix(satori_hip_matrix* m) {
    m->q8k.release();
    m->planes.release();
    if (m->payload) (void)hipFree(m->payload);
    if (m->scratch) (void)hipFree(m->scratch);
    m->payload = nullptr;
    m->scratch = nullptr;
}

// A device matrix holding `payload` (already checked against the shape) in its device layout. A Ternary2 payload
// (or, with `bitplanes`, a ternary bitplane payload, converted to its Ternary2 equivalent) is checked on the
// device as it is regrouped; one that breaks the rule is named by the host restatement of
// Ternary2Matrix.ValidatePayload (TernaryBitplaneMatrix.Validate), which throws the reference's error (the device
// copy is freed first).
satori_hip_matrix* upload(satori_hip_context* c, const Shape& s, const uint8_t* payload, bool bitplanes = false) {
    require_not_capturing(c);
    set_device(c);
    const int64_t bytes = device_layout_bytes(s);
    auto* m = new satori_hip_matrix();
    m->context = c;
    m->shape = s;
    bool valid = true;
    try {
        allocate_matrix(m, bytes);
        valid = upload_layout(c, s, payload, m->payload, bitplanes);
        check_hip(hipMemset(m->payload + bytes, 0, kPayloadSlack), "weight upload");
    } catch (...) {
        free_matrix(m);
        delete m;
        throw;
    }
    if (!valid) {
        free_matrix(m);
        delete m;
        if (bitplanes) {
            validate_bitplane(s, payload);
            fail(SATORI_HIP_E_ARGUMENT, "Overlapping bits, invalid padding or noncanonical zero. (Parameter 'data')");
        }
        validate_ternary2(s, payload);
        fail(SATORI_HIP_E_ARGUMENT, "Invalid weight code or padding.");
    }
    c->matrices++;
    return m;
}

// upload() of a GGUF-format payload whose block scales are then checked on the device (QuantizedMatVec's
// finiteness rule, scale_check.hip). A payload that fails is named by the host restatement of the rule
// (validate_quantized), which throws the reference's error with the first bad block's offset.
satori_hip_matrix* upload_checked(satori_hip_context* c, const Shape& s, const uint8_t* payload) {
    satori_hip_matrix* m = upload(c, s, payload);
    uint32_t bad = 0;
    try {
        c->upload_flag.reserve(sizeof(uint32_t));
        uint32_t* flag = static_cast<uint32_t*>(c->upload_flag.ptr);
        check_hip(hipMemsetAsync(flag, 0, sizeof(uint32_t), c->stream), "scale check");
        check_hip(launch_scale_check(m->payload, static_cast<int64_t>(s.rows) * s.blocks, s.format, flag, c->stream),
                  "scale check");
        check_hip(hipMemcpyAsync(&bad, flag, sizeof(bad), hipMemcpyDeviceToHost, c->stream), "scale check");
        check_hip(hipStreamSynchronize(c->stream), "scale check");
    } catch (...) {
        free_matrix(m);
        delete m;
        c->matrices--;
        throw;
    }
    if (bad != 0) {
        free_matrix(m);
        delete m;
        c->matrices--;
        validate_quantized(s, payload);  // names the first bad block
        fail(SATORI_HIP_E_INVALID_DATA, "Nonfinite block scale.");
    }
    return m;
}

// Host-buffer MatVec shared by matvec and matvec_batch.
// A host-buffer call's vector between its pinned staging buffer and the device, on the context stream: up to
// kKernelCopyMaxBytes by a copy kernel over the host link, larger ones by the copy engine.
void move_vector(satori_hip_context* c, const void* src, void* dst, size_t bytes, hipMemcpyKind kind,
                 const char* what) {
    if (bytes <= kKernelCopyMaxBytes)
        check_hip(launch_copy_words(src, dst, bytes, c->stream), what);
    else
        check_hip(hipMemcpyAsync(dst, src, bytes, kind, c->stream), what);
}

void host_matvec(satori_hip_matrix* m, const float* input, size_t input_length, int positions, float* output,
                 size_t output_length, bool batch) {
    require(m, "matrix");
    satori_hip_context* c = m->context;
    std::lock_guard<std::mutex> guard(c->lock);
    require_live(m);
    require_not_capturing(c);
    require(input, "input");
    require(output, "output");
    const Shape& s = m->shape;
    if (batch) {
        if (positions <= 0) fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "positions must be positive.");
        if (s.format == SATORI_HIP_TERNARY2)
            fail(SATORI_HIP_E_NOT_SUPPORTED, "The batched product is defined for the GGUF block formats only.");
        const int64_t in_need = static_cast<int64_t>(positions) * s.columns;
        const int64_t out_need = static_cast<int64_t>(positions) * s.rows;
        if (in_need > INT32_MAX || out_need > INT32_MAX)
            fail(SATORI_HIP_E_OVERFLOW, "Arithmetic operation resulted in an overflow.");
        if (static_cast<int64_t>(input_length) != in_need)
            fail(SATORI_HIP_E_ARGUMENT, "Input must hold one vector per position.");
        if (static_cast<int64_t>(output_length) != out_need)
            fail(SATORI_HIP_E_ARGUMENT, "Output must hold one vector per position.");
        if (is_k(s) && positions > 256)
            fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "At most 256 positions per call.");
    } else {
        positions = 1;
        if (input_length != static_cast<size_t>(s.columns) || output_length != static_cast<size_t>(s.rows))
            fail(SATORI_HIP_E_ARGUMENT, "Vector lengths must match matrix dimensions.");
    }
    const size_t in_bytes = input_length * sizeof(float), out_bytes = output_length * sizeof(float);
    if (overlaps(input, in_bytes, output, out_bytes))
        fail(SATORI_HIP_E_ARGUMENT, "Output must not overlap input.");
    // Only the plugin seam rejects non-finite activations: IQuantizedMatrix.Execute of a GPU backend
    // (src/Satori.Backends.Vulkan/VulkanQ8Matrix.cs:82-83). Ternary2MatVec.Execute (Ternary2MatVec.cs:30-36)
    // and QuantizedMatVec.ExecuteBatch (QuantizedMatVec.cs:104-116) take them and propagate them.
    if (!batch && s.format != SATORI_HIP_TERNARY2)
        for (size_t i = 0; i < input_length; ++i)
            if (!std::isfinite(input[i])) fail(SATORI_HIP_E_ARGUMENT, "Expected finite FP32 input.");

    set_device(c);
    c->x.reserve(in_bytes);
    c->host_x.reserve(in_bytes);
    c->host_y.reserve(out_bytes);
    const bool integer = batch && is_k(s);
    std::memcpy(c->host_x.ptr, input, in_bytes);
    move_vector(c, c->host_x.ptr, c->x.ptr, in_bytes, hipMemcpyHostToDevice, "input copy");
    // The product kernels store each output element once (no read-back, no atomics on y), so outputs of up
    // to kKernelCopyMaxBytes are written straight into the pinned output staging buffer over the host link;
    // larger ones (many-position batches) go to device memory and then through the copy engine.
    const bool direct = out_bytes <= kKernelCopyMaxBytes;
    if (!direct) c->y.reserve(out_bytes);
    float* y = static_cast<float*>(direct ? c->host_y.ptr : c->y.ptr);
    if (integer)
        enqueue_kint(m, static_cast<const float*>(c->x.ptr), positions, y, c->stream);
    else
        enqueue_float(m, static_cast<const float*>(c->x.ptr), positions, y, c->stream);
    if (!direct)
        check_hip(hipMemcpyAsync(c->host_y.ptr, c->y.ptr, out_bytes, hipMemcpyDeviceToHost, c->stream), "output copy");
    check_hip(hipStreamSynchronize(c->stream), "stream");
    std::memcpy(output, c->host_y.ptr, out_bytes);  // commit only after success
}

// Enqueues one group's launch on `st`.
void enqueue_group(satori_hip_group* g, hipStream_t st) {
    const LaunchShape l = launch_shape(g->shape, 1, g->rows_max);
    const MatDesc none{};
    if (g->quantized && g->output.activated) {
        check_hip(launch_gemv_kint_swiglu(g->host.data(), l, g->input, g->output, st), "integer gemv launch");
    } else if (g->quantized && g->input.kind != kInputPlain) {
        check_hip(launch_gemv_kint_transformed(g->host.data(), g->descriptors, g->count, l, g->input, st),
                  "integer gemv launch");
    } else if (g->quantized && g->shared_q8k.ptr) {
        // One input shared by many members: quantized once by a small launch, each workgroup copies its bytes
        // (the same bytes every workgroup would compute).
        check_hip(launch_q8k_quantize(g->host[0].x, g->shape.columns, 1, static_cast<uint8_t*>(g->shared_q8k.ptr), st),
                  "Q8_K quantization launch");
        InputTransform t{};
        t.kind = kInputQ8K;
        t.a = static_cast<const float*>(g->shared_q8k.ptr);
        check_hip(launch_gemv_kint_transformed(g->host.data(), g->descriptors, g->count, l, t, st),
                  "integer gemv launch");
    } else if (g->quantized) {
        check_hip(launch_gemv_kint(g->host.data(), g->descriptors, g->count, l, st), "integer gemv launch");
    } else if (g->shape.format == SATORI_HIP_TERNARY2) {
        check_hip(launch_t2(none, g->descriptors, g->count, l, g->plan, g->scratch, next_t2_generation(g->t2_generation),
                            st),
                  "Ternary2 launch");
    } else {
        check_hip(launch_gemv_float(none, g->descriptors, g->count, l, st), "gemv launch");
    }
}

// Enqueues one K-format group over `positions` positions (inputs [positions][columns], outputs
// [positions][rows]): the integer kernel below kmfma_min_positions(), else the matrix-core product, with the
// Q8_K pack of each distinct input pointer done once and up to kKmfmaMaxMembers members per launch.
void enqueue_group_batch(satori_hip_group* g, int positions, hipStream_t st) {
    const Shape& s = g->shape;
    if (g->input.kind != kInputPlain)
        fail(SATORI_HIP_E_NOT_SUPPORTED, "An input transform applies to one-position group launches only.");
    if (g->output.activated)
        fail(SATORI_HIP_E_NOT_SUPPORTED, "An output transform applies to one-position group launches only.");
    if (positions < kmfma_min_positions()) {
        check_hip(launch_gemv_kint(g->host.data(), g->descriptors, g->count, launch_shape(s, positions, g->rows_max), st),
                  "integer gemv launch");
        return;
    }
    std::vector<const float*> inputs;
    std::vector<size_t> slot(g->count);
    for (int i = 0; i < g->count; ++i) {
        auto it = std::find(inputs.begin(), inputs.end(), g->host[i].x);
        slot[i] = static_cast<size_t>(it - inputs.begin());
        if (it == inputs.end()) inputs.push_back(g->host[i].x);
    }
    const size_t per = kmfma_workspace_bytes(s.blocks, positions);
    if (g->context->capturing && g->batch.bytes < per * inputs.size())
        fail(SATORI_HIP_E_INVALID_OPERATION,
             "Run this many-position product once before capturing it (its workspace is allocated on first use).");
    if (g->steps > 0 && g->batch.bytes < per * inputs.size())  // a captured step holds the current buffer
        fail(SATORI_HIP_E_INVALID_OPERATION,
             "The workspace of this group cannot grow while a captured step replays it: destroy the step, "
             "or run the largest product before capturing.");
    // Each member's weight planes (the member matrix of descriptor i is the one whose payload it reads).
    std::vector<const uint8_t*> planes(g->count);
    for (int i = 0; i < g->count; ++i) {
        satori_hip_matrix* owner = nullptr;
        for (satori_hip_matrix* m : g->members)
            if (m->payload == g->host[i].w) owner = m;
        if (!owner) fail(SATORI_HIP_E_INVALID_OPERATION, "Group member not found.");
        planes[i] = ensure_planes(owner, st);
    }
    g->batch.reserve(per * inputs.size());
    uint8_t* ws = static_cast<uint8_t*>(g->batch.ptr);
    for (size_t k = 0; k < inputs.size(); ++k)
        check_hip(launch_kmfma_pack(s.format, inputs[k], s.blocks, positions, ws + k * per, st), "Q8_K pack launch");
    for (int i0 = 0; i0 < g->count; i0 += kKmfmaMaxMembers) {
        const int n = std::min(kKmfmaMaxMembers, g->count - i0);
        KmfmaMember members[kKmfmaMaxMembers];
        for (int j = 0; j < n; ++j) {
            const MatDesc& d = g->host[i0 + j];
            members[j] = KmfmaMember{planes[i0 + j], ws + slot[i0 + j] * per, d.y, d.rows, 0, s.row_bytes};
        }
        check_hip(launch_kmfma_product(s.format, members, n, s.blocks, positions, st), "matrix-core gemv launch");
    }
}

// A whole file mapped read-only for the duration of a call.
struct MappedFile {
    const uint8_t* bytes = nullptr;
    size_t length = 0;
    explicit MappedFile(const char* path) {
        const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
        if (fd < 0) fail(SATORI_HIP_E_ARGUMENT, std::string("Cannot open ") + path + ".");
        struct stat st;
        if (::fstat(fd, &st) != 0) {
            ::close(fd);
            fail(SATORI_HIP_E_ARGUMENT, std::string("Cannot stat ") + path + ".");
        }
        length = static_cast<size_t>(st.st_size);
        if (length > 0) {
            void* map = ::mmap(nullptr, length, PROT_READ, MAP_PRIVATE, fd, 0);
            if (map == MAP_FAILED) {
                ::close(fd);
                fail(SATORI_HIP_E_ARGUMENT, std::string("Cannot map ") + path + ".");
            }
            bytes = static_cast<const uint8_t*>(map);
        }
        ::close(fd);
    }
    ~MappedFile() {
        if (bytes) ::munmap(const_cast<uint8_t*>(bytes), length);
    }
};

// TernaryBitplaneMatrix.Load (src/Satori.Core/TernaryBitplaneMatrix.cs:98-117) with
// TernaryBitplaneFileFormat.ReadHeader (src/Satori.Core/TernaryBitplaneFileFormat.cs:13-19): the STQ2 header
// with magic "STB1"; every failure is InvalidDataException. Returns the shape of a valid file.
// MappedTernaryBitplaneMatrix: shape and payload failures of a file surface as InvalidDataException.
[[noreturn]] void bitplane_file_failure(const Failure& e) {
    if (e.status == SATORI_HIP_E_ARGUMENT || e.status == SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE ||
        e.status == SATORI_HIP_E_OVERFLOW)
        fail(SATORI_HIP_E_INVALID_DATA, "Invalid bitplane file.");
    throw e;
}

// Shape of an STB1 file; its payload is validated here only when `validate` (an upload validates it on the
// device instead, bitplane_file_failure naming its failures as this function does).
Shape read_bitplane_file(const MappedFile& f, bool validate = true) {
    if (f.length < 32) fail(SATORI_HIP_E_INVALID_DATA, "Truncated bitplane header.");
    const uint8_t* h = f.bytes;
    if (std::memcmp(h, "STB1", 4) != 0) fail(SATORI_HIP_E_INVALID_DATA, "Invalid bitplane magic.");
    int32_t rows, columns, block, reserved;
    int64_t declared;
    std::memcpy(&rows, h + 8, 4);
    std::memcpy(&columns, h + 12, 4);
    std::memcpy(&block, h + 16, 4);
    std::memcpy(&reserved, h + 20, 4);
    std::memcpy(&declared, h + 24, 8);
    if (u16_at(h + 4) != 1 || u16_at(h + 6) != 32 || reserved != 0)
        fail(SATORI_HIP_E_INVALID_DATA, "Invalid bitplane header fields.");
    Shape s;
    try {
        s = ternary2_shape(rows, columns, block);
        if (declared != s.byte_length) fail(SATORI_HIP_E_INVALID_DATA, "Invalid bitplane header fields.");
        if (static_cast<int64_t>(f.length) != 32 + s.byte_length)
            fail(SATORI_HIP_E_INVALID_DATA, "Incorrect bitplane file length.");
        if (validate) validate_bitplane(s, h + 32);
    } catch (const Failure& e) {
        bitplane_file_failure(e);
    }
    return s;
}

// A bitplane payload executes as its lossless Ternary2 equivalent (same bytes per block, same scales): upload()
// converts and validates it on the device.
satori_hip_matrix* upload_bitplane(satori_hip_context* c, const Shape& s, const uint8_t* payload) {
    return upload(c, s, payload, true);
}

const satori::GgufFile& live_file(const satori_hip_gguf* f) {
    require(f, "file");
    if (!f->live) fail(SATORI_HIP_E_OBJECT_DISPOSED, "Cannot access a disposed object. Object name: 'GgufFile'.");
    return *f->file;
}

const GgufTensorInfo& tensor_at(const GgufFile& file, int64_t index) {
    if (index < 0 || index >= static_cast<int64_t>(file.tensors().size()))
        fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "Tensor index out of range. (Parameter 'index')");
    return file.tensors()[static_cast<size_t>(index)];
}

const GgufMetadataInfo& metadata_at(const GgufFile& file, int64_t index) {
    if (index < 0 || index >= static_cast<int64_t>(file.metadata().size()))
        fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "Metadata index out of range. (Parameter 'index')");
    return file.metadata()[static_cast<size_t>(index)];
}

void require_live(const satori_hip_group* g) {
    require(g, "group");
    if (!g->live || !g->context->live)
        fail(SATORI_HIP_E_OBJECT_DISPOSED, "Cannot access a disposed object. Object name: 'satori_hip_group'.");
}

}  // namespace
}  // namespace satori

using namespace satori;

extern "C" {

int satori_hip_abi_version(void) { return SATORI_HIP_ABI_VERSION; }

const char* satori_hip_last_error(void) { return g_last_error.c_str(); }

int satori_hip_device_count(int* count) {
    return guarded([&] {
        require(count, "count");
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
        int gfx950 = 0;
        for (int i = 0; i < n; ++i) {
            hipDeviceProp_t prop;
            if (hipGetDeviceProperties(&prop, i) == hipSuccess && std::strncmp(prop.gcnArchName, "gfx950", 6) == 0)
                gfx950++;
        }
        *count = gfx950;
    });
}

int satori_hip_context_create(int device, satori_hip_context** context) {
    return guarded([&] {
        require(context, "context");
        *context = nullptr;
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess || n == 0)
            fail(SATORI_HIP_E_PLATFORM_NOT_SUPPORTED, "No HIP device is available.");
        if (device < 0 || device >= n) fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "device is out of range.");
        hipDeviceProp_t prop;
        check_hip(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
        if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
            fail(SATORI_HIP_E_PLATFORM_NOT_SUPPORTED, std::string("Device is ") + prop.gcnArchName + ", not gfx950.");
        check_hip(hipSetDevice(device), "hipSetDevice");
        double* partials = nullptr;
        check_hip(static_attention_partials(&partials), "hipGetSymbolAddress");  // with `device` current
        auto* c = new satori_hip_context();
        c->device = device;
        c->static_attention = partials;
        const hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
        if (e != hipSuccess) {
            delete c;
            check_hip(e, "hipStreamCreate");
        }
        *context = c;
    });
}

int satori_hip_context_destroy(satori_hip_context* c) {
    return guarded([&] {
        if (!c) return;
        std::lock_guard<std::mutex> guard(c->lock);
        require_not_capturing(c);
        if (!c->live) return;
        if (c->matrices > 0)
            fail(SATORI_HIP_E_ARGUMENT, "Matrices created on the context must be destroyed first.");
        (void)hipSetDevice(c->device);
        (void)hipStreamSynchronize(c->stream);
        c->x.release();
        c->y.release();
        c->q8k.release();
        c->upload_stage.release();
        c->upload_flag.release();
        for (auto& entry : c->attention) entry.second.release();
        c->attention.clear();
        c->host_x.release();
        c->host_y.release();
        (void)hipStreamDestroy(c->stream);
        c->stream = nullptr;
        c->live = false;  // the handle stays valid as a tombstone so a second destroy is a no-op
    });
}

int satori_hip_context_stream(satori_hip_context* c, void** stream) {
    return guarded([&] {
        require_live(c);
        require(stream, "stream");
        *stream = c->stream;
    });
}

int satori_hip_ternary2_create(satori_hip_context* c, int rows, int columns, int block_size, const void* payload,
                               size_t payload_length, satori_hip_matrix** matrix) {
    return guarded([&] {
        require(matrix, "matrix");
        *matrix = nullptr;
        require_live(c);
        const Shape s = ternary2_shape(rows, columns, block_size);
        require(payload, "payload");
        if (static_cast<int64_t>(payload_length) != s.byte_length)
            fail(SATORI_HIP_E_ARGUMENT, "Payload length must match matrix dimensions.");
        std::lock_guard<std::mutex> guard(c->lock);
        require_live(c);
        *matrix = upload(c, s, static_cast<const uint8_t*>(payload));  // validates the payload as it regroups it
    });
}

int satori_hip_quantized_create(satori_hip_context* c, int rows, int columns, int format, const void* payload,
                                size_t payload_length, satori_hip_matrix** matrix) {
    return guarded([&] {
        require(matrix, "matrix");
        *matrix = nullptr;
        require_live(c);
        const Shape s = quantized_shape(rows, columns, format);
        require(payload, "payload");
        if (static_cast<int64_t>(payload_length) != s.byte_length)
            fail(SATORI_HIP_E_ARGUMENT, "Incorrect quantized payload length.");
        std::lock_guard<std::mutex> guard(c->lock);
        require_live(c);
        *matrix = upload_checked(c, s, static_cast<const uint8_t*>(payload));  // scales checked on the device
    });
}

int satori_hip_ternary2_open(satori_hip_context* c, const char* path, satori_hip_matrix** matrix) {
    return guarded([&] {
        require(matrix, "matrix");
        *matrix = nullptr;
        require_live(c);
        require(path, "path");
        const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
        if (fd < 0) fail(SATORI_HIP_E_ARGUMENT, std::string("Cannot open ") + path + ".");
        struct stat st;
        if (::fstat(fd, &st) != 0) {
            ::close(fd);
            fail(SATORI_HIP_E_ARGUMENT, std::string("Cannot stat ") + path + ".");
        }
        const size_t length = static_cast<size_t>(st.st_size);
        if (length < 32) {
            ::close(fd);
            fail(SATORI_HIP_E_INVALID_DATA, "Truncated Ternary2 header.");  // MappedTernary2Matrix.cs:14-15
        }
        void* map = ::mmap(nullptr, length, PROT_READ, MAP_PRIVATE, fd, 0);
        ::close(fd);
        if (map == MAP_FAILED) fail(SATORI_HIP_E_ARGUMENT, std::string("Cannot map ") + path + ".");
        struct Unmap {
            void* p;
            size_t n;
            ~Unmap() { ::munmap(p, n); }
        } unmap{map, length};
        const uint8_t* h = static_cast<const uint8_t*>(map);
        // Ternary2FileFormat.ReadHeader (src/Satori.Core/Ternary2FileFormat.cs:21-35).
        int32_t rows, columns, block, reserved;
        int64_t declared;
        std::memcpy(&rows, h + 8, 4);
        std::memcpy(&columns, h + 12, 4);
        std::memcpy(&block, h + 16, 4);
        std::memcpy(&reserved, h + 20, 4);
        std::memcpy(&declared, h + 24, 8);
        if (std::memcmp(h, "STQ2", 4) != 0 || u16_at(h + 4) != 1 || u16_at(h + 6) != 32 || reserved != 0)
            fail(SATORI_HIP_E_INVALID_DATA, "Unsupported Ternary2 header.");
        Shape s;
        try {
            s = ternary2_shape(rows, columns, block);
            if (declared != s.byte_length) fail(SATORI_HIP_E_INVALID_DATA, "Payload length disagrees with matrix shape.");
            if (static_cast<int64_t>(length) != 32 + s.byte_length)
                fail(SATORI_HIP_E_INVALID_DATA, "Truncated payload or trailing file data.");
            std::lock_guard<std::mutex> guard(c->lock);
            require_live(c);
            *matrix = upload(c, s, h + 32);  // validates the payload as it regroups it
        } catch (const Failure& f) {
            // MappedTernary2Matrix.cs:25-28: shape and payload failures surface as InvalidDataException.
            if (f.status == SATORI_HIP_E_ARGUMENT || f.status == SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE ||
                f.status == SATORI_HIP_E_OVERFLOW)
                fail(SATORI_HIP_E_INVALID_DATA, "Invalid Ternary2 shape or payload.");
            throw;
        }
    });
}

int satori_hip_bitplane_create(satori_hip_context* c, int rows, int columns, int block_size, const void* payload,
                               size_t payload_length, satori_hip_matrix** matrix) {
    return guarded([&] {
        require(matrix, "matrix");
        *matrix = nullptr;
        require_live(c);
        const Shape s = ternary2_shape(rows, columns, block_size);
        require(payload, "payload");
        if (static_cast<int64_t>(payload_length) != s.byte_length)
            fail(SATORI_HIP_E_ARGUMENT, "Incorrect bitplane payload length. (Parameter 'payload')");
        std::lock_guard<std::mutex> guard(c->lock);
        require_live(c);
        *matrix = upload_bitplane(c, s, static_cast<const uint8_t*>(payload));  // validates as it converts
    });
}

int satori_hip_bitplane_open(satori_hip_context* c, const char* path, satori_hip_matrix** matrix) {
    return guarded([&] {
        require(matrix, "matrix");
        *matrix = nullptr;
        require_live(c);
        require(path, "path");
        MappedFile f(path);
        const Shape s = read_bitplane_file(f, false);
        std::lock_guard<std::mutex> guard(c->lock);
        require_live(c);
        try {
            *matrix = upload_bitplane(c, s, f.bytes + 32);  // validates the payload as it converts it
        } catch (const Failure& e) {
            bitplane_file_failure(e);
        }
    });
}

int satori_hip_bitplane_load(const char* path, int* rows, int* columns, int* block_size, void* payload,
                             size_t capacity, int64_t* length) {
    return guarded([&] {
        require(path, "path");
        MappedFile f(path);
        const Shape s = read_bitplane_file(f);
        if (rows) *rows = s.rows;
        if (columns) *columns = s.columns;
        if (block_size) *block_size = s.block_size;
        if (length) *length = s.byte_length;
        if (payload) {
            if (static_cast<int64_t>(capacity) < s.byte_length)
                fail(SATORI_HIP_E_ARGUMENT, "Destination is too short. (Parameter 'payload')");
            std::memcpy(payload, f.bytes + 32, static_cast<size_t>(s.byte_length));
        }
    });
}

int satori_hip_matrix_clone(satori_hip_matrix* source, satori_hip_matrix** clone) {
    return guarded([&] {
        require(clone, "clone");
        *clone = nullptr;
        require(source, "source");
        satori_hip_context* c = source->context;
        std::lock_guard<std::mutex> guard(c->lock);
        require_not_capturing(c);
        require_live(source);
        set_device(c);
        auto* m = new satori_hip_matrix();
        m->context = c;
        m->shape = source->shape;
        try {
            allocate_matrix(m, source->device_bytes);
            const size_t bytes = static_cast<size_t>(source->device_bytes) + kPayloadSlack;
            check_hip(hipMemcpyAsync(m->payload, source->payload, bytes, hipMemcpyDeviceToDevice, c->stream),
                      "clone copy");
            check_hip(hipStreamSynchronize(c->stream), "clone copy");
        } catch (...) {
            free_matrix(m);
            delete m;
            throw;
        }
        c->matrices++;
        *clone = m;
    });
}

int satori_hip_matrix_destroy(satori_hip_matrix* m) {
    return guarded([&] {
        if (!m) return;
        satori_hip_context* c = m->context;
        std::lock_guard<std::mutex> guard(c->lock);
        require_not_capturing(c);
        if (!m->live) return;
        if (m->groups > 0) fail(SATORI_HIP_E_ARGUMENT, "Groups that launch the matrix must be destroyed first.");
        if (c->live) {
            (void)hipSetDevice(c->device);
            (void)hipStreamSynchronize(c->stream);
        }
        free_matrix(m);
        m->live = false;  // tombstone: later calls report ObjectDisposed, a second destroy is a no-op
        c->matrices--;
    });
}

int satori_hip_matrix_shape(const satori_hip_matrix* m, int* rows, int* columns, int* format, int* block_size,
                            int64_t* byte_length) {
    return guarded([&] {
        require_live(m);
        if (rows) *rows = m->shape.rows;
        if (columns) *columns = m->shape.columns;
        if (format) *format = m->shape.format;
        if (block_size) *block_size = m->shape.block_size;
        if (byte_length) *byte_length = m->shape.byte_length;
    });
}

int satori_hip_matvec(satori_hip_matrix* m, const float* input, size_t input_length, float* output,
                      size_t output_length) {
    return guarded([&] { host_matvec(m, input, input_length, 1, output, output_length, false); });
}

int satori_hip_matvec_batch(satori_hip_matrix* m, const float* input, size_t input_length, int positions,
                            float* output, size_t output_length) {
    return guarded([&] { host_matvec(m, input, input_length, positions, output, output_length, true); });
}

int satori_hip_quantize_q8k(satori_hip_context* c, const float* input, int columns, void* output,
                            size_t output_length) {
    return guarded([&] {
        require_live(c);
        require(input, "input");
        require(output, "output");
        if (columns <= 0 || columns % 256 != 0)
            fail(SATORI_HIP_E_ARGUMENT, "Invalid Q8_K row dimensions.");  // Q8KCodec.QuantizeRow, :88-89
        const size_t out_bytes = static_cast<size_t>(columns / 256) * kQ8KBlockBytes;
        if (output_length != out_bytes) fail(SATORI_HIP_E_ARGUMENT, "Invalid Q8_K row dimensions.");
        const size_t in_bytes = static_cast<size_t>(columns) * sizeof(float);
        std::lock_guard<std::mutex> guard(c->lock);
        require_not_capturing(c);
        require_live(c);
        set_device(c);
        c->x.reserve(in_bytes);
        c->q8k.reserve(out_bytes);
        c->host_x.reserve(in_bytes);
        c->host_y.reserve(out_bytes);
        std::memcpy(c->host_x.ptr, input, in_bytes);
        move_vector(c, c->host_x.ptr, c->x.ptr, in_bytes, hipMemcpyHostToDevice, "input copy");
        check_hip(launch_q8k_quantize(static_cast<const float*>(c->x.ptr), columns, 1,
                                      static_cast<uint8_t*>(c->q8k.ptr), c->stream),
                  "Q8_K launch");
        move_vector(c, c->q8k.ptr, c->host_y.ptr, out_bytes, hipMemcpyDeviceToHost, "output copy");
        check_hip(hipStreamSynchronize(c->stream), "stream");
        std::memcpy(output, c->host_y.ptr, out_bytes);
    });
}

int satori_hip_matvec_device(satori_hip_matrix* m, const float* input, float* output, void* stream) {
    return guarded([&] {
        require(m, "matrix");
        std::lock_guard<std::mutex> guard(m->context->lock);
        require_live(m);
        require(input, "input");
        require(output, "output");
        set_device(m->context);
        const hipStream_t st = stream ? static_cast<hipStream_t>(stream) : m->context->stream;
        enqueue_float(m, input, 1, output, st);
        note_launch(m->context, m, st);
    });
}

int satori_hip_matvec_batch_device(satori_hip_matrix* m, const float* input, int positions, float* output,
                                   void* stream) {
    return guarded([&] {
        require(m, "matrix");
        satori_hip_context* c = m->context;
        std::lock_guard<std::mutex> guard(c->lock);
        require_live(m);
        require(input, "input");
        require(output, "output");
        if (positions <= 0) fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "positions must be positive.");
        if (m->shape.format == SATORI_HIP_TERNARY2)
            fail(SATORI_HIP_E_NOT_SUPPORTED, "The batched product is defined for the GGUF block formats only.");
        set_device(c);
        hipStream_t st = stream ? static_cast<hipStream_t>(stream) : c->stream;
        if (is_k(m->shape)) {
            if (positions > 256) fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "At most 256 positions per call.");
            enqueue_kint(m, input, positions, output, st);
        } else {
            enqueue_float(m, input, positions, output, st);
        }
        note_launch(c, m, st);
    });
}

int satori_hip_device_alloc(satori_hip_context* c, size_t bytes, void** device_ptr) {
    return guarded([&] {
        require(device_ptr, "device_ptr");
        *device_ptr = nullptr;
        require_live(c);
        std::lock_guard<std::mutex> guard(c->lock);
        require_not_capturing(c);
        if (bytes == 0) fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "bytes must be positive.");
        set_device(c);
        check_hip(hipMalloc(device_ptr, bytes), "hipMalloc");
    });
}

int satori_hip_device_free(satori_hip_context* c, void* device_ptr) {
    return guarded([&] {
        require_live(c);
        std::lock_guard<std::mutex> guard(c->lock);
        require_not_capturing(c);
        if (!device_ptr) return;
        set_device(c);
        check_hip(hipStreamSynchronize(c->stream), "stream");
        check_hip(hipFree(device_ptr), "hipFree");
    });
}

int satori_hip_copy(satori_hip_context* c, void* destination, const void* source, size_t bytes, int kind) {
    return guarded([&] {
        require_live(c);
        require(destination, "destination");
        require(source, "source");
        hipMemcpyKind k;
        switch (kind) {
            case 1: k = hipMemcpyHostToDevice; break;
            case 2: k = hipMemcpyDeviceToHost; break;
            case 3: k = hipMemcpyDeviceToDevice; break;
            default: fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "kind must be 1, 2 or 3.");
        }
        std::lock_guard<std::mutex> guard(c->lock);
        require_not_capturing(c);
        set_device(c);
        check_hip(hipMemcpyAsync(destination, source, bytes, k, c->stream), "hipMemcpyAsync");
        check_hip(hipStreamSynchronize(c->stream), "stream");
    });
}

int satori_hip_synchronize(satori_hip_context* c) {
    return guarded([&] {
        require_live(c);
        std::lock_guard<std::mutex> guard(c->lock);
        require_not_capturing(c);
        set_device(c);
        check_hip(hipStreamSynchronize(c->stream), "stream");
    });
}

int satori_hip_group_create(satori_hip_context* c, satori_hip_matrix* const* matrices, int count,
                            const float* const* inputs, float* const* outputs, int quantized_activations,
                            satori_hip_group** group) {
    return guarded([&] {
        require(group, "group");
        *group = nullptr;
        require_live(c);
        require(matrices, "matrices");
        require(inputs, "inputs");
        require(outputs, "outputs");
        if (count <= 0) fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "count must be positive.");
        std::lock_guard<std::mutex> guard(c->lock);
        require_not_capturing(c);
        const Shape& first = matrices[0] ? matrices[0]->shape : Shape{};
        std::vector<MatDesc> host(count);
        auto* g = new satori_hip_group();
        g->context = c;
        g->count = count;
        try {
            for (int i = 0; i < count; ++i) {
                require_live(matrices[i]);
                if (matrices[i]->context != c) fail(SATORI_HIP_E_ARGUMENT, "Every member must belong to the context.");
                const Shape& s = matrices[i]->shape;
                if (s.format != first.format || s.columns != first.columns || s.block_size != first.block_size)
                    fail(SATORI_HIP_E_ARGUMENT, "Group members must share format, block size and column count.");
                require(inputs[i], "inputs[i]");
                require(outputs[i], "outputs[i]");
                host[i] = MatDesc{matrices[i]->payload, inputs[i], outputs[i], s.rows, 0};
                g->rows_max = std::max(g->rows_max, s.rows);
            }
            g->shape = first;
            g->quantized = quantized_activations != 0 && is_k(first);
            if (first.format == SATORI_HIP_TERNARY2) {
                g->plan = t2_plan(g->rows_max, first.columns, first.block_size, count, 1);
                set_device(c);
                g->scratch = allocate_t2_scratch(g->plan);
            }
            set_device(c);
            // Groups of more members than a launch passes in its arguments (large launches that stream from HBM)
            // whose members all read one input of more than 16 blocks quantize it once per launch instead of in
            // every workgroup (a workgroup quantizes 16 blocks per pass: 1536 x 8960 grouped, Q4_K 5.65 -> 5.83
            // TB/s, Q6_K 5.82 -> 5.89; for rows of one pass the extra launch cost more, 8960 x 1536 -2%).
            bool shared_input = true;
            for (int i = 1; i < count; ++i) shared_input = shared_input && host[i].x == host[0].x;
            if (g->quantized && count > kKintInlineMembers && shared_input && first.columns / 256 > 16)
                g->shared_q8k.reserve(static_cast<size_t>(first.columns / 256) * kQ8KBlockBytes);
            check_hip(hipMalloc(reinterpret_cast<void**>(&g->descriptors), sizeof(MatDesc) * count), "hipMalloc");
            check_hip(hipMemcpy(g->descriptors, host.data(), sizeof(MatDesc) * count, hipMemcpyHostToDevice),
                      "descriptor upload");
            g->host = host;
        } catch (...) {
            if (g->descriptors) (void)hipFree(g->descriptors);
            if (g->scratch) (void)hipFree(g->scratch);
            g->shared_q8k.release();
            delete g;
            throw;
        }
        for (int i = 0; i < count; ++i)
            if (std::find(g->members.begin(), g->members.end(), matrices[i]) == g->members.end()) {
                g->members.push_back(matrices[i]);
                matrices[i]->groups++;
            }
        *group = g;
    });
}

int satori_hip_group_execute(satori_hip_group* g, void* stream) {
    return guarded([&] {
        require(g, "group");
        satori_hip_context* c = g->context;
        std::lock_guard<std::mutex> guard(c->lock);
        if (!g->live || !c->live) fail(SATORI_HIP_E_OBJECT_DISPOSED, "Cannot access a disposed object. Object name: 'satori_hip_group'.");
        set_device(c);
        const hipStream_t st = stream ? static_cast<hipStream_t>(stream) : c->stream;
        enqueue_group(g, st);
        if (c->capturing && st == c->stream) c->captured_groups.push_back(g);
    });
}

int satori_hip_group_execute_batch(satori_hip_group* g, int positions, void* stream) {
    return guarded([&] {
        require(g, "group");
        satori_hip_context* c = g->context;
        std::lock_guard<std::mutex> guard(c->lock);
        if (!g->live || !c->live) fail(SATORI_HIP_E_OBJECT_DISPOSED, "Cannot access a disposed object. Object name: 'satori_hip_group'.");
        if (!g->quantized)
            fail(SATORI_HIP_E_NOT_SUPPORTED,
                 "The many-position group product is defined for K-format groups with quantized activations.");
        if (positions <= 0 || positions > 256) fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "positions must be 1..256.");
        set_device(c);
        const hipStream_t st = stream ? static_cast<hipStream_t>(stream) : c->stream;
        enqueue_group_batch(g, positions, st);
        if (c->capturing && st == c->stream) c->captured_groups.push_back(g);
    });
}

int satori_hip_group_set_input(satori_hip_group* g, int kind, const float* a, const float* b, const float* weights,
                               float epsilon, float* residual_out) {
    return guarded([&] {
        require(g, "group");
        satori_hip_context* c = g->context;
        std::lock_guard<std::mutex> guard(c->lock);
        if (!g->live || !c->live) fail(SATORI_HIP_E_OBJECT_DISPOSED, "Cannot access a disposed object. Object name: 'satori_hip_group'.");
        require_not_capturing(c);
        if (g->steps > 0) fail(SATORI_HIP_E_ARGUMENT, "Steps that replay the group must be destroyed first.");
        if (!g->quantized)
            fail(SATORI_HIP_E_NOT_SUPPORTED, "Input transforms apply to K-format groups with quantized activations.");
        InputTransform t{};
        t.kind = kind;
        switch (kind) {
            case SATORI_HIP_INPUT_PLAIN: break;
            case SATORI_HIP_INPUT_ADD_RMS_NORM:
                require(a, "a");
                require(weights, "weights");
                // The operator's own rule (TransformerOps.cs:17): epsilon finite and positive.
                if (!std::isfinite(epsilon) || epsilon <= 0.0f)
                    fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE,
                         "Specified argument was out of the range of valid values. (Parameter 'epsilon')");
                break;
            case SATORI_HIP_INPUT_SWIGLU:
                require(a, "a");
                require(b, "b");
                if (g->output.activated)
                    fail(SATORI_HIP_E_NOT_SUPPORTED, "The SwiGlu input transform does not combine with the SwiGlu output.");
                break;
            case SATORI_HIP_INPUT_Q8K:
                require(a, "a");
                break;
            default: fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "Unknown input transform.");
        }
        if (kind != SATORI_HIP_INPUT_PLAIN) {
            t.a = a;
            t.b = kind == SATORI_HIP_INPUT_Q8K ? nullptr : b;
            t.w = kind == SATORI_HIP_INPUT_ADD_RMS_NORM ? weights : nullptr;
            t.epsilon = epsilon;
            t.residual_out = kind == SATORI_HIP_INPUT_ADD_RMS_NORM ? residual_out : nullptr;
            const size_t n = static_cast<size_t>(g->shape.columns) * sizeof(float);
            if (t.residual_out) {
                // One workgroup writes residual_out while the others read the operands and write the outputs.
                bool clash = overlaps(t.residual_out, n, a, n) || (b && overlaps(t.residual_out, n, b, n)) ||
                             overlaps(t.residual_out, n, weights, n);
                for (const MatDesc& d : g->host)
                    clash = clash || overlaps(t.residual_out, n, d.y, static_cast<size_t>(d.rows) * sizeof(float));
                if (clash) fail(SATORI_HIP_E_ARGUMENT, "residual_out must not overlap the operands or the outputs.");
            }
        }
        if (g->output.activated) {  // the SwiGlu output's buffers, written by the launch that reads t's operands
            const int rows = g->host[0].rows;
            const size_t act_bytes = static_cast<size_t>(rows) * sizeof(float);
            const size_t q_bytes = g->output.q8k ? static_cast<size_t>(rows / 256) * kQ8KBlockBytes : 0;
            if (overlaps_transform(g->output.activated, act_bytes, t, g->shape.columns) ||
                (q_bytes && overlaps_transform(g->output.q8k, q_bytes, t, g->shape.columns)))
                fail(SATORI_HIP_E_ARGUMENT, "The input transform's buffers must not overlap activated or q8k.");
        }
        g->input = t;
    });
}

int satori_hip_group_set_output(satori_hip_group* g, int kind, float* activated, void* q8k) {
    return guarded([&] {
        require(g, "group");
        satori_hip_context* c = g->context;
        std::lock_guard<std::mutex> guard(c->lock);
        if (!g->live || !c->live) fail(SATORI_HIP_E_OBJECT_DISPOSED, "Cannot access a disposed object. Object name: 'satori_hip_group'.");
        require_not_capturing(c);
        if (g->steps > 0) fail(SATORI_HIP_E_ARGUMENT, "Steps that replay the group must be destroyed first.");
        if (kind == SATORI_HIP_OUTPUT_PLAIN) {
            set_device(c);
            check_hip(hipStreamSynchronize(c->stream), "stream");  // no launch still counts into the buffer
            g->output = OutputSwiGluQ8K{};
            g->counters.release();
            return;
        }
        if (kind != SATORI_HIP_OUTPUT_SWIGLU) fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "Unknown output transform.");
        if (!g->quantized)
            fail(SATORI_HIP_E_NOT_SUPPORTED, "Output transforms apply to K-format groups with quantized activations.");
        require(activated, "activated");
        if (g->count != 2 || g->host[0].rows != g->host[1].rows)
            fail(SATORI_HIP_E_ARGUMENT, "The SwiGlu output needs two members (gate, up) with the same row count.");
        if (g->input.kind == kInputSwiGlu)
            fail(SATORI_HIP_E_NOT_SUPPORTED, "The SwiGlu output does not combine with the SwiGlu input transform.");
        const int rows = g->host[0].rows;
        if (rows % 256 != 0)
            fail(SATORI_HIP_E_ARGUMENT, "The SwiGlu output is quantized to Q8_K: the row count must be a multiple of 256.");
        const size_t act_bytes = static_cast<size_t>(rows) * sizeof(float);
        const size_t q_bytes = q8k ? static_cast<size_t>(rows / 256) * kQ8KBlockBytes : 0;
        const size_t in_bytes = static_cast<size_t>(g->shape.columns) * sizeof(float);
        bool clash = overlaps(activated, act_bytes, q8k, q_bytes);
        for (const MatDesc& d : g->host)
            clash = clash || overlaps(activated, act_bytes, d.y, act_bytes) || overlaps(q8k, q_bytes, d.y, act_bytes) ||
                    overlaps(activated, act_bytes, d.x, in_bytes) || overlaps(q8k, q_bytes, d.x, in_bytes);
        // With an input transform the launch reads its operands (and may write residual_out) instead of x.
        clash = clash || overlaps_transform(activated, act_bytes, g->input, g->shape.columns) ||
                (q_bytes && overlaps_transform(q8k, q_bytes, g->input, g->shape.columns));
        if (clash) fail(SATORI_HIP_E_ARGUMENT, "activated and q8k must not overlap each other, the inputs or the outputs.");
        set_device(c);
        check_hip(hipStreamSynchronize(c->stream), "stream");
        if (q8k) {
            g->counters.reserve(static_cast<size_t>(rows / 256) * sizeof(uint32_t));
            check_hip(hipMemset(g->counters.ptr, 0, g->counters.bytes), "counter clear");
        } else {
            g->counters.release();
        }
        g->output = OutputSwiGluQ8K{activated, static_cast<uint8_t*>(q8k),
                                    q8k ? static_cast<uint32_t*>(g->counters.ptr) : nullptr};
    });
}

int satori_hip_group_destroy(satori_hip_group* g) {
    return guarded([&] {
        if (!g) return;
        satori_hip_context* c = g->context;
        std::lock_guard<std::mutex> guard(c->lock);
        require_not_capturing(c);
        if (!g->live) return;
        if (g->steps > 0) fail(SATORI_HIP_E_ARGUMENT, "Steps that replay the group must be destroyed first.");
        if (c->live) {
            (void)hipSetDevice(c->device);
            (void)hipStreamSynchronize(c->stream);
        }
        for (satori_hip_matrix* m : g->members) m->groups--;
        g->members.clear();
        (void)hipFree(g->descriptors);
        g->descriptors = nullptr;
        if (g->scratch) (void)hipFree(g->scratch);
        g->scratch = nullptr;
        g->batch.release();
        g->counters.release();
        g->shared_q8k.release();
        g->output = OutputSwiGluQ8K{};
        g->live = false;
    });
}

int satori_hip_step_create(satori_hip_context* c, satori_hip_group* const* groups, int count,
                           satori_hip_step** step) {
    return guarded([&] {
        require(step, "step");
        *step = nullptr;
        require_live(c);
        require(groups, "groups");
        if (count <= 0) fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "count must be positive.");
        std::lock_guard<std::mutex> guard(c->lock);
        require_not_capturing(c);
        for (int i = 0; i < count; ++i) {
            require_live(groups[i]);
            if (groups[i]->context != c) fail(SATORI_HIP_E_ARGUMENT, "Every group must belong to the context.");
        }
        set_device(c);
        // Everything enqueued on the context stream before the capture must not be part of the graph.
        check_hip(hipStreamSynchronize(c->stream), "stream");
        check_hip(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal), "graph capture");
        hipGraph_t graph = nullptr;
        try {
            for (int i = 0; i < count; ++i) enqueue_group(groups[i], c->stream);
        } catch (...) {
            (void)hipStreamEndCapture(c->stream, &graph);
            if (graph) (void)hipGraphDestroy(graph);
            throw;
        }
        check_hip(hipStreamEndCapture(c->stream, &graph), "graph capture");
        hipGraphExec_t exec = nullptr;
        const hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        if (e != hipSuccess) {
            (void)hipGraphDestroy(graph);
            check_hip(e, "graph instantiation");
        }
        auto* s = new satori_hip_step();
        s->context = c;
        s->graph = graph;
        s->exec = exec;
        s->groups.assign(groups, groups + count);
        for (satori_hip_group* g : s->groups) g->steps++;
        *step = s;
    });
}

int satori_hip_step_execute(satori_hip_step* s, void* stream) {
    return guarded([&] {
        require(s, "step");
        satori_hip_context* c = s->context;
        std::lock_guard<std::mutex> guard(c->lock);
        require_not_capturing(c);
        if (!s->live || !c->live)
            fail(SATORI_HIP_E_OBJECT_DISPOSED, "Cannot access a disposed object. Object name: 'satori_hip_step'.");
        set_device(c);
        check_hip(hipGraphLaunch(s->exec, stream ? static_cast<hipStream_t>(stream) : c->stream), "graph launch");
    });
}

int satori_hip_step_destroy(satori_hip_step* s) {
    return guarded([&] {
        if (!s) return;
        satori_hip_context* c = s->context;
        std::lock_guard<std::mutex> guard(c->lock);
        require_not_capturing(c);
        if (!s->live) return;
        if (c->live) {
            (void)hipSetDevice(c->device);
            (void)hipStreamSynchronize(c->stream);
        }
        (void)hipGraphExecDestroy(s->exec);
        (void)hipGraphDestroy(s->graph);
        s->exec = nullptr;
        s->graph = nullptr;
        for (satori_hip_group* g : s->groups) g->steps--;
        for (satori_hip_matrix* m : s->matrices) {
            m->groups--;
            m->steps--;
        }
        if (s->attention) c->attention_steps--;
        s->attention = false;
        s->groups.clear();
        s->matrices.clear();
        s->live = false;
    });
}

int satori_hip_capture_begin(satori_hip_context* c) {
    return guarded([&] {
        require_live(c);
        std::lock_guard<std::mutex> guard(c->lock);
        require_live(c);
        require_not_capturing(c);
        set_device(c);
        // Everything enqueued on the context stream before the capture must not be part of the graph.
        check_hip(hipStreamSynchronize(c->stream), "stream");
        check_hip(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal), "graph capture");
        c->capturing = true;
        c->captured_matrices.clear();
        c->captured_groups.clear();
        c->captured_attention = false;
    });
}

int satori_hip_capture_end(satori_hip_context* c, satori_hip_step** step) {
    return guarded([&] {
        require(step, "step");
        *step = nullptr;
        require_live(c);
        std::lock_guard<std::mutex> guard(c->lock);
        if (!c->capturing) fail(SATORI_HIP_E_INVALID_OPERATION, "The context stream is not being captured.");
        set_device(c);
        c->capturing = false;
        std::vector<satori_hip_matrix*> matrices;
        std::vector<satori_hip_group*> groups;
        matrices.swap(c->captured_matrices);
        groups.swap(c->captured_groups);
        hipGraph_t graph = nullptr;
        check_hip(hipStreamEndCapture(c->stream, &graph), "graph capture");
        if (!graph) fail(SATORI_HIP_E_DEVICE, "The capture produced no graph.");
        hipGraphExec_t exec = nullptr;
        const hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        if (e != hipSuccess) {
            (void)hipGraphDestroy(graph);
            check_hip(e, "graph instantiation");
        }
        auto* st = new satori_hip_step();
        st->context = c;
        st->graph = graph;
        st->exec = exec;
        for (satori_hip_group* g : groups) {
            if (std::find(st->groups.begin(), st->groups.end(), g) == st->groups.end()) {
                st->groups.push_back(g);
                g->steps++;
            }
        }
        for (satori_hip_matrix* m : matrices) {
            if (std::find(st->matrices.begin(), st->matrices.end(), m) == st->matrices.end()) {
                st->matrices.push_back(m);
                m->groups++;
                m->steps++;
            }
        }
        st->attention = c->captured_attention;
        if (st->attention) c->attention_steps++;
        c->captured_attention = false;
        *step = st;
    });
}

// ---- GGUF containers ----

int satori_hip_gguf_open(const char* path, satori_hip_gguf** file) {
    return guarded([&] {
        require(file, "file");
        *file = nullptr;
        require(path, "path");
        auto* parsed = new GgufFile(path);
        *file = new satori_hip_gguf{parsed, true};
    });
}

int satori_hip_gguf_close(satori_hip_gguf* file) {
    return guarded([&] {
        if (!file || !file->live) return;
        delete file->file;
        file->file = nullptr;
        file->live = false;
    });
}

int satori_hip_gguf_data_offset(const satori_hip_gguf* file, int64_t* offset) {
    return guarded([&] {
        const GgufFile& f = live_file(file);
        require(offset, "offset");
        *offset = f.data_offset();
    });
}

int satori_hip_gguf_tensor_count(const satori_hip_gguf* file, int64_t* count) {
    return guarded([&] {
        const GgufFile& f = live_file(file);
        require(count, "count");
        *count = static_cast<int64_t>(f.tensors().size());
    });
}

int satori_hip_gguf_tensor_find(const satori_hip_gguf* file, const char* name, int64_t* index) {
    return guarded([&] {
        const GgufFile& f = live_file(file);
        require(name, "name");
        require(index, "index");
        const int64_t k = f.find_tensor(name);
        if (k < 0) fail(SATORI_HIP_E_KEY_NOT_FOUND, std::string("The given key '") + name + "' was not present in the dictionary.");
        *index = k;
    });
}

int satori_hip_gguf_tensor_info(const satori_hip_gguf* file, int64_t index, const char** name, int* rank,
                                int64_t dims[4], uint32_t* type, int64_t* offset, int64_t* byte_length) {
    return guarded([&] {
        const GgufTensorInfo& t = tensor_at(live_file(file), index);
        if (name) *name = t.name.c_str();
        if (rank) *rank = t.rank;
        if (dims)
            for (int d = 0; d < 4; ++d) dims[d] = t.dims[d];
        if (type) *type = t.type;
        if (offset) *offset = t.offset;
        if (byte_length) *byte_length = t.byte_length;
    });
}

int satori_hip_gguf_tensor_window(const satori_hip_gguf* file, int64_t index, int64_t offset, int64_t length,
                                  const void** bytes) {
    return guarded([&] {
        const GgufFile& f = live_file(file);
        const GgufTensorInfo& t = tensor_at(f, index);
        require(bytes, "bytes");
        // GgufFile.cs:44-46.
        if (offset < 0 || length < 0 || offset > t.byte_length || length > t.byte_length - offset)
            fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "Window exceeds tensor payload. (Parameter 'offset')");
        *bytes = f.bytes() + t.offset + offset;
    });
}

int satori_hip_gguf_metadata_count(const satori_hip_gguf* file, int64_t* count) {
    return guarded([&] {
        const GgufFile& f = live_file(file);
        require(count, "count");
        *count = static_cast<int64_t>(f.metadata().size());
    });
}

int satori_hip_gguf_metadata_find(const satori_hip_gguf* file, const char* key, int64_t* index) {
    return guarded([&] {
        const GgufFile& f = live_file(file);
        require(key, "key");
        require(index, "index");
        const int64_t k = f.find_metadata(key);
        if (k < 0) fail(SATORI_HIP_E_KEY_NOT_FOUND, std::string("The given key '") + key + "' was not present in the dictionary.");
        *index = k;
    });
}

int satori_hip_gguf_metadata_info(const satori_hip_gguf* file, int64_t index, const char** key, uint32_t* type,
                                  int64_t* offset, int64_t* byte_length, int64_t* element_type,
                                  int64_t* element_count) {
    return guarded([&] {
        const GgufMetadataInfo& m = metadata_at(live_file(file), index);
        if (key) *key = m.key.c_str();
        if (type) *type = m.type;
        if (offset) *offset = m.offset;
        if (byte_length) *byte_length = m.byte_length;
        if (element_type) *element_type = m.element_type;
        if (element_count) *element_count = m.element_count;
    });
}

int satori_hip_gguf_metadata_window(const satori_hip_gguf* file, int64_t index, const void** bytes, int64_t* length) {
    return guarded([&] {
        const GgufFile& f = live_file(file);
        const GgufMetadataInfo& m = metadata_at(f, index);
        require(bytes, "bytes");
        // GgufFile.cs:54.
        if (m.byte_length > 0x7FFFFFFF) fail(SATORI_HIP_E_NOT_SUPPORTED, "Metadata window exceeds Int32.");
        *bytes = f.bytes() + m.offset;
        if (length) *length = m.byte_length;
    });
}

int satori_hip_gguf_matrix_create(satori_hip_context* c, const satori_hip_gguf* file, int64_t index,
                                  satori_hip_matrix** matrix) {
    return guarded([&] {
        require(matrix, "matrix");
        *matrix = nullptr;
        require_live(c);
        const GgufFile& f = live_file(file);
        const GgufTensorInfo& t = tensor_at(f, index);
        // GgufQuantizedMatrix.cs:16-26.
        const bool typed = t.type == 8 || t.type == 2 || t.type == 12 || t.type == 14;
        if (!typed || t.rank != 2 || t.byte_length > 0x7FFFFFFF || t.dims[0] > 0x7FFFFFFF || t.dims[1] > 0x7FFFFFFF)
            fail(SATORI_HIP_E_NOT_SUPPORTED,
                 "MatVec requires a rank-2 Q8_0/Q4_0/Q4_K/Q6_K tensor within Int32 limits.");
        const int format = t.type == 8 ? SATORI_HIP_Q8_0 : t.type == 2 ? SATORI_HIP_Q4_0
                           : t.type == 12 ? SATORI_HIP_Q4_K : SATORI_HIP_Q6_K;
        const Shape s = quantized_shape(static_cast<int>(t.dims[1]), static_cast<int>(t.dims[0]), format);
        const uint8_t* bytes = f.bytes() + t.offset;  // the whole payload: ReadTensor(name, 0, ByteLength)
        std::lock_guard<std::mutex> guard(c->lock);
        require_live(c);
        *matrix = upload_checked(c, s, bytes);
    });
}

// ---- decode-step operators (TransformerOps, src/Satori.Core/TransformerOps.cs), device pointers ----

}  // extern "C"

namespace {

// Ranges [a, a + n) and [b, b + m) of floats overlap without starting at the same element.
bool partial_overlap(const void* a, int64_t n, const void* b, int64_t m) {
    const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
    const bool overlap = x < y + static_cast<uintptr_t>(m) * 4 && y < x + static_cast<uintptr_t>(n) * 4;
    return overlap && x != y;
}

bool any_overlap(const void* a, int64_t n, const void* b, int64_t m) {
    const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
    return n > 0 && m > 0 && x < y + static_cast<uintptr_t>(m) * 4 && y < x + static_cast<uintptr_t>(n) * 4;
}

hipStream_t op_stream(satori_hip_context* c, void* stream) {
    return stream ? static_cast<hipStream_t>(stream) : c->stream;
}

// Entry-point frame of the operators: context checks and lock, device current, status from the launch.
template <class F>
int op_call(satori_hip_context* c, F&& body) {
    return guarded([&] {
        require_live(c);
        std::lock_guard<std::mutex> guard(c->lock);
        require_live(c);
        set_device(c);
        body();
    });
}

void check_epsilon(float epsilon) {
    if (!std::isfinite(epsilon) || epsilon <= 0)
        fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "Specified argument was out of the range of valid values. (Parameter 'epsilon')");
}

}  // namespace

extern "C" {

int satori_hip_rms_norm(satori_hip_context* c, const float* input, const float* weights, float epsilon, int length,
                        int count, float* output, void* stream) {
    return op_call(c, [&] {
        require(input, "input");
        require(weights, "weights");
        require(output, "output");
        if (length <= 0 || count <= 0) fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "Specified argument was out of the range of valid values. (Parameter 'epsilon')");
        check_epsilon(epsilon);
        const int64_t n = static_cast<int64_t>(length) * count;
        if (partial_overlap(input, n, output, n) || any_overlap(weights, length, output, n))
            fail(SATORI_HIP_E_ARGUMENT, "Partial overlap.");
        check_hip(launch_rms_norm(input, weights, epsilon, length, count, output, op_stream(c, stream)), "rms_norm launch");
    });
}

int satori_hip_rms_norm_heads(satori_hip_context* c, float* vector, const float* weights, float epsilon, int head_dim,
                              int length, void* stream) {
    return op_call(c, [&] {
        require(vector, "vector");
        require(weights, "weights");
        if (head_dim <= 0 || length <= 0 || length % head_dim != 0)
            fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "Specified argument was out of the range of valid values. (Parameter 'headDimension')");
        check_epsilon(epsilon);
        if (any_overlap(weights, head_dim, vector, length)) fail(SATORI_HIP_E_ARGUMENT, "Partial overlap.");
        check_hip(launch_rms_norm_heads(vector, weights, epsilon, head_dim, length / head_dim, op_stream(c, stream)),
                  "rms_norm_heads launch");
    });
}

int satori_hip_rope(satori_hip_context* c, float* vector, int length, int head_dim, int position, void* stream) {
    return op_call(c, [&] {
        require(vector, "vector");
        if (head_dim <= 0 || head_dim % 2 != 0 || length <= 0 || length % head_dim != 0 || position < 0)
            fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "Specified argument was out of the range of valid values. (Parameter 'headDimension')");
        check_hip(launch_rope(vector, length / head_dim, head_dim, position, 10000.0, head_dim, false, op_stream(c, stream)),
                  "rope launch");
    });
}

int satori_hip_rope_half(satori_hip_context* c, float* vector, int length, int head_dim, int position,
                         double frequency_base, int rotary_dimensions, void* stream) {
    return op_call(c, [&] {
        require(vector, "vector");
        if (head_dim <= 0 || length <= 0 || length % head_dim != 0 || position < 0)
            fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "Specified argument was out of the range of valid values. (Parameter 'headDimension')");
        if (!std::isfinite(frequency_base) || frequency_base <= 0)
            fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "Specified argument was out of the range of valid values. (Parameter 'frequencyBase')");
        if (rotary_dimensions <= 0 || rotary_dimensions > head_dim || rotary_dimensions % 2 != 0)
            fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "Specified argument was out of the range of valid values. (Parameter 'rotaryDimensions')");
        check_hip(launch_rope(vector, length / head_dim, head_dim, position, frequency_base, rotary_dimensions, true,
                              op_stream(c, stream)),
                  "rope_half launch");
    });
}

int satori_hip_swiglu(satori_hip_context* c, const float* gate, const float* up, int length, float* output,
                      void* stream) {
    return op_call(c, [&] {
        require(gate, "gate");
        require(up, "up");
        require(output, "output");
        if (length < 0) fail(SATORI_HIP_E_ARGUMENT, "Lengths differ.");
        if (partial_overlap(gate, length, output, length) || partial_overlap(up, length, output, length))
            fail(SATORI_HIP_E_ARGUMENT, "Partial overlap.");
        if (length > 0) check_hip(launch_swiglu(gate, up, length, output, op_stream(c, stream)), "swiglu launch");
    });
}

int satori_hip_swiglu_q8k(satori_hip_context* c, const float* gate, const float* up, int length, float* output,
                          void* q8k, void* stream) {
    return op_call(c, [&] {
        require(gate, "gate");
        require(up, "up");
        require(q8k, "q8k");
        if (length <= 0 || length % 256 != 0) fail(SATORI_HIP_E_ARGUMENT, "Invalid Q8_K row dimensions.");
        if (output && (partial_overlap(gate, length, output, length) || partial_overlap(up, length, output, length)))
            fail(SATORI_HIP_E_ARGUMENT, "Partial overlap.");
        const int64_t q_floats = static_cast<int64_t>(length / 256) * kQ8KBlockBytes / 4;
        if (any_overlap(q8k, q_floats, gate, length) || any_overlap(q8k, q_floats, up, length) ||
            (output && any_overlap(q8k, q_floats, output, length)))
            fail(SATORI_HIP_E_ARGUMENT, "Partial overlap.");
        check_hip(launch_swiglu_q8k(gate, up, length, output, static_cast<uint8_t*>(q8k), op_stream(c, stream)),
                  "swiglu launch");
    });
}

int satori_hip_quantize_q8k_device(satori_hip_context* c, const float* input, int columns, int positions, void* output,
                                   void* stream) {
    return op_call(c, [&] {
        require(input, "input");
        require(output, "output");
        if (columns <= 0 || columns % 256 != 0) fail(SATORI_HIP_E_ARGUMENT, "Invalid Q8_K row dimensions.");
        if (positions <= 0) fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "positions must be positive.");
        const int64_t n = static_cast<int64_t>(columns) * positions;
        if (any_overlap(output, n / 256 * kQ8KBlockBytes / 4, input, n)) fail(SATORI_HIP_E_ARGUMENT, "Partial overlap.");
        check_hip(launch_q8k_quantize(input, columns, positions, static_cast<uint8_t*>(output), op_stream(c, stream)),
                  "Q8_K launch");
    });
}

int satori_hip_add(satori_hip_context* c, const float* left, const float* right, int length, float* output,
                   void* stream) {
    return op_call(c, [&] {
        require(left, "left");
        require(right, "right");
        require(output, "output");
        if (length < 0) fail(SATORI_HIP_E_ARGUMENT, "Lengths differ.");
        if (partial_overlap(left, length, output, length) || partial_overlap(right, length, output, length))
            fail(SATORI_HIP_E_ARGUMENT, "Partial overlap.");
        if (length > 0) check_hip(launch_add(left, right, length, output, op_stream(c, stream)), "add launch");
    });
}

int satori_hip_add_rms_norm(satori_hip_context* c, float* residual, const float* addend, const float* weights,
                            float epsilon, int length, float* normed, void* stream) {
    return op_call(c, [&] {
        require(residual, "residual");
        require(addend, "addend");
        require(weights, "weights");
        require(normed, "normed");
        if (length <= 0) fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "Specified argument was out of the range of valid values. (Parameter 'epsilon')");
        check_epsilon(epsilon);
        if (partial_overlap(addend, length, residual, length) || any_overlap(normed, length, residual, length) ||
            any_overlap(weights, length, normed, length) || any_overlap(addend, length, normed, length))
            fail(SATORI_HIP_E_ARGUMENT, "Partial overlap.");
        check_hip(launch_add_rms_norm(residual, addend, weights, epsilon, length, normed, op_stream(c, stream)),
                  "add_rms_norm launch");
    });
}

int satori_hip_add_rms_norm_q8k(satori_hip_context* c, float* residual, const float* addend, const float* weights,
                                float epsilon, int length, float* normed, void* q8k, void* stream) {
    return op_call(c, [&] {
        require(residual, "residual");
        require(addend, "addend");
        require(weights, "weights");
        require(normed, "normed");
        require(q8k, "q8k");
        if (length <= 0 || length % 256 != 0) fail(SATORI_HIP_E_ARGUMENT, "Invalid Q8_K row dimensions.");
        check_epsilon(epsilon);
        const int64_t q_floats = static_cast<int64_t>(length / 256) * kQ8KBlockBytes / 4;
        if (partial_overlap(addend, length, residual, length) || any_overlap(normed, length, residual, length) ||
            any_overlap(weights, length, normed, length) || any_overlap(addend, length, normed, length) ||
            any_overlap(q8k, q_floats, residual, length) || any_overlap(q8k, q_floats, addend, length) ||
            any_overlap(q8k, q_floats, weights, length) || any_overlap(q8k, q_floats, normed, length))
            fail(SATORI_HIP_E_ARGUMENT, "Partial overlap.");
        check_hip(launch_add_rms_norm_q8k(residual, addend, weights, epsilon, length, normed,
                                          static_cast<uint8_t*>(q8k), op_stream(c, stream)),
                  "add_rms_norm_q8k launch");
    });
}

int satori_hip_attention_inputs(satori_hip_context* c, float* query, const float* query_bias, const float* key,
                                const float* key_bias, float* key_out, const float* value, const float* value_bias,
                                float* value_out, int query_heads, int kv_heads, int head_dim, int position,
                                double frequency_base, int rotary_dimensions, void* stream) {
    return op_call(c, [&] {
        require(query, "query");
        require(key, "key");
        require(key_out, "keyOut");
        require(value, "value");
        require(value_out, "valueOut");
        if (head_dim <= 0 || query_heads <= 0 || kv_heads <= 0 || position < 0)
            fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "Specified argument was out of the range of valid values. (Parameter 'headDimension')");
        if (!std::isfinite(frequency_base) || frequency_base <= 0)
            fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "Specified argument was out of the range of valid values. (Parameter 'frequencyBase')");
        if (rotary_dimensions <= 0 || rotary_dimensions > head_dim || rotary_dimensions % 2 != 0)
            fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "Specified argument was out of the range of valid values. (Parameter 'rotaryDimensions')");
        const int64_t qw = static_cast<int64_t>(query_heads) * head_dim, kw = static_cast<int64_t>(kv_heads) * head_dim;
        if (any_overlap(key, kw, key_out, kw) && key != key_out) fail(SATORI_HIP_E_ARGUMENT, "Partial overlap.");
        if (any_overlap(value, kw, value_out, kw) && value != value_out) fail(SATORI_HIP_E_ARGUMENT, "Partial overlap.");
        if (any_overlap(query, qw, key_out, kw) || any_overlap(query, qw, value_out, kw) ||
            any_overlap(key_out, kw, value_out, kw))
            fail(SATORI_HIP_E_ARGUMENT, "Partial overlap.");
        check_hip(launch_attention_inputs(query, query_bias, key, key_bias, key_out, value, value_bias, value_out,
                                          query_heads, kv_heads, head_dim, position, frequency_base, rotary_dimensions,
                                          op_stream(c, stream)),
                  "attention_inputs launch");
    });
}

}  // extern "C"

namespace {

// GroupedAttention's argument rules (TransformerOps.cs:135-145), shared by both attention entry points.
void check_attention(const float* query, const float* keys, const float* values, int query_heads, int kv_heads,
                     int head_dim, int tokens, float* output) {
    require(query, "query");
    require(keys, "keys");
    require(values, "values");
    require(output, "output");
    if (head_dim <= 0 || query_heads <= 0 || kv_heads <= 0 || query_heads % kv_heads != 0 || tokens <= 0)
        fail(SATORI_HIP_E_ARGUMENT, "Invalid grouped-attention dimensions.");
    const int64_t width = static_cast<int64_t>(query_heads) * head_dim;
    const int64_t kv = static_cast<int64_t>(tokens) * kv_heads * head_dim;
    if (width > INT32_MAX || kv > INT32_MAX) fail(SATORI_HIP_E_OVERFLOW, "Arithmetic operation resulted in an overflow.");
    if (any_overlap(query, width, output, width) || any_overlap(keys, kv, output, width) ||
        any_overlap(values, kv, output, width))
        fail(SATORI_HIP_E_ARGUMENT, "Attention output overlaps input.");
    if (!attention_supported(tokens, head_dim))
        fail(SATORI_HIP_E_NOT_SUPPORTED, "The prefix is too long for one split of the attention's local memory.");
}

// The split attention's partials for a call on stream `st`: the context's buffer for that stream, allocated by
// its first split attention and grown as prefixes grow (not while capturing, nor while captured steps hold the
// context stream's buffer); null when the call needs none.
double* attention_workspace(satori_hip_context* c, hipStream_t st, int query_heads, int head_dim, int tokens) {
    if (attention_splits(tokens) <= 1) return nullptr;
    const size_t need = attention_scratch_bytes(query_heads, head_dim, tokens);
    auto it = std::find_if(c->attention.begin(), c->attention.end(),
                           [&](const std::pair<hipStream_t, DeviceBuffer>& e) { return e.first == st; });
    if (c->capturing && (it == c->attention.end() || it->second.bytes < need))
        fail(SATORI_HIP_E_INVALID_OPERATION,
             "Run an attention of these heads and tokens once before capturing it (its workspace is allocated "
             "on first use).");
    if (it == c->attention.end()) {
        c->attention.emplace_back(st, DeviceBuffer{});
        it = c->attention.end() - 1;
    }
    DeviceBuffer& buffer = it->second;
    if (st == c->stream && c->attention_steps > 0 && buffer.bytes < need)  // captured steps hold it
        fail(SATORI_HIP_E_INVALID_OPERATION,
             "The attention workspace cannot grow while captured steps use it: destroy them, or run the "
             "longest attention before capturing.");
    buffer.reserve(need);
    if (c->capturing && st == c->stream) c->captured_attention = true;
    return static_cast<double*>(buffer.ptr);
}

}  // namespace

extern "C" {

int satori_hip_grouped_attention(satori_hip_context* c, const float* query, const float* keys, const float* values,
                                 int query_heads, int kv_heads, int head_dim, int tokens, float* output, void* stream) {
    return op_call(c, [&] {
        check_attention(query, keys, values, query_heads, kv_heads, head_dim, tokens, output);
        const hipStream_t st = op_stream(c, stream);
        double* scratch = attention_workspace(c, st, query_heads, head_dim, tokens);
        check_hip(launch_attention(query, keys, values, query_heads, kv_heads, head_dim, tokens, output, scratch, st),
                  "attention launch");
    });
}

int satori_hip_attention_decode(satori_hip_context* c, float* query, const float* query_bias, const float* key,
                                const float* key_bias, const float* value, const float* value_bias, float* keys,
                                float* values, int query_heads, int kv_heads, int head_dim, int position,
                                double frequency_base, int rotary_dimensions, const double* rope_table, float* output,
                                void* stream) {
    return op_call(c, [&] {
        require(key, "key");
        require(value, "value");
        if (head_dim <= 0 || query_heads <= 0 || kv_heads <= 0 || position < 0)
            fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "Specified argument was out of the range of valid values. (Parameter 'headDimension')");
        if (!std::isfinite(frequency_base) || frequency_base <= 0)
            fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "Specified argument was out of the range of valid values. (Parameter 'frequencyBase')");
        if (rotary_dimensions <= 0 || rotary_dimensions > head_dim || rotary_dimensions % 2 != 0)
            fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "Specified argument was out of the range of valid values. (Parameter 'rotaryDimensions')");
        if (position == INT32_MAX) fail(SATORI_HIP_E_OVERFLOW, "Arithmetic operation resulted in an overflow.");
        check_attention(query, keys, values, query_heads, kv_heads, head_dim, position + 1, output);
        const int64_t qw = static_cast<int64_t>(query_heads) * head_dim, kw = static_cast<int64_t>(kv_heads) * head_dim;
        const int64_t cache = (static_cast<int64_t>(position) + 1) * kw;
        // The inputs and the cache must not overlap one another or the query and output (the launch reads the
        // new key and value while it writes row `position` of the cache).
        if (any_overlap(key, kw, keys, cache) || any_overlap(key, kw, values, cache) ||
            any_overlap(value, kw, keys, cache) || any_overlap(value, kw, values, cache) ||
            any_overlap(query, qw, keys, cache) || any_overlap(query, qw, values, cache) ||
            any_overlap(keys, cache, values, cache) || any_overlap(key, kw, output, qw) ||
            any_overlap(value, kw, output, qw))
            fail(SATORI_HIP_E_ARGUMENT, "Partial overlap.");
        const hipStream_t st = op_stream(c, stream);
        double* scratch = attention_workspace(c, st, query_heads, head_dim, position + 1);
        const double* rope = rope_table ? rope_table + static_cast<int64_t>(position) * rotary_dimensions : nullptr;
        check_hip(launch_attention_decode(query, query_bias, key, key_bias, value, value_bias, keys, values, query_heads,
                                          kv_heads, head_dim, position, frequency_base, rotary_dimensions, rope, output,
                                          scratch, st),
                  "attention launch");
    });
}

int satori_hip_rope_table(satori_hip_context* c, int positions, int rotary_dimensions, double frequency_base,
                          double* table, void* stream) {
    return op_call(c, [&] {
        require(table, "table");
        if (positions <= 0) fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "positions must be positive.");
        if (!std::isfinite(frequency_base) || frequency_base <= 0)
            fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "Specified argument was out of the range of valid values. (Parameter 'frequencyBase')");
        if (rotary_dimensions <= 0 || rotary_dimensions % 2 != 0)
            fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "Specified argument was out of the range of valid values. (Parameter 'rotaryDimensions')");
        check_hip(launch_rope_table(positions, rotary_dimensions, frequency_base, table, op_stream(c, stream)),
                  "rope table launch");
    });
}

int satori_hip_grouped_attention_static(satori_hip_context* c, const float* query, const float* keys,
                                        const float* values, int query_heads, int kv_heads, int head_dim, int tokens,
                                        float* output, void* stream) {
    return op_call(c, [&] {
        check_attention(query, keys, values, query_heads, kv_heads, head_dim, tokens, output);
        const size_t need = attention_partials_bytes(query_heads, head_dim, tokens);
        if (need > kStaticAttentionBytes)
            fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE,
                 "The attention needs " + std::to_string(need) + " bytes of partials (query_heads * splits * "
                 "(head_dim + 2) * 8); the static workspace holds " + std::to_string(kStaticAttentionBytes) + ".");
        // No workspace to allocate or grow: the partials (written in full before the combine reads them, so
        // nothing needs clearing) go to the device's static array.
        check_hip(launch_attention(query, keys, values, query_heads, kv_heads, head_dim, tokens, output,
                                   c->static_attention, op_stream(c, stream)),
                  "attention launch");
    });
}

int satori_hip_matrix_decode_row(satori_hip_matrix* m, int row, float* output, void* stream) {
    return guarded([&] {
        require(m, "matrix");
        satori_hip_context* c = m->context;
        std::lock_guard<std::mutex> guard(c->lock);
        require_live(m);
        require(output, "output");
        const Shape& s = m->shape;
        if (s.format == SATORI_HIP_Q4_0) fail(SATORI_HIP_E_NOT_SUPPORTED, "Q4_0 embedding rows are not supported.");
        if (s.format == SATORI_HIP_TERNARY2) fail(SATORI_HIP_E_NOT_SUPPORTED, "Embedding rows are defined for the GGUF block formats.");
        if (row < 0 || row >= s.rows)
            fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "Specified argument was out of the range of valid values. (Parameter 'row')");
        set_device(c);
        check_hip(launch_decode_row(m->payload, s.format, s.rows, s.columns, row, output, op_stream(c, stream)),
                  "decode_row launch");
        note_launch(c, m, op_stream(c, stream));
    });
}

}  // extern "C"
