// refmodel.hip — reference-model mode: the reference's own network
// (backend-cuda.cu:23-54) behind the same field interface as the hash-grid
// model.
//
//   encoding   frequency encoding of the world position, 10 levels, and of the
//              ray direction, 4 levels (:252-277): [x, y, z, then per level
//              sin x, sin y, sin z, cos x, cos y, cos z]
//   density    64 (63 encoded values and a zero, :918-927) -> 128 -> 128 x 4
//              -> 16, ReLU between layers, no biases
//   colour     48 = [raw density outputs 1..15 | direction encoding (27) |
//              0 x 6] (:928-943) -> 128 -> 128 x 2 -> 16 (3 used)
//   outputs    sigma = softplus(raw density 0) (:913-917), rgb = sigmoid
//              (:910-912)
//
// Rounding points: fp16 inputs, fp16 hidden activations, fp16 raw outputs
// (the reference's output buffers are fp16); MFMA accumulation in fp32.
//
// Layout.  A layer computes out^T = W . in^T on v_mfma_f32_16x16x32_f16 with
// 16 output rows of W as the A operand and 16 samples as the B operand, as the
// hash-grid model's MLPs do: a layer's fp32 results, rounded to fp16 and
// ReLU'd, are directly the next layer's B operand when the next layer's
// weights are read with the matching k-permutation (KMap::Hidden).  The 128 x
// 128 layers do not fit in registers or LDS (232 KiB of weights in all), so
// the weights are packed once per call into A-fragment order — fragment
// (row block r, k-block q) is 64 lanes x 8 halves = 1 KiB, contiguous — and
// every A fragment is one coalesced 16-byte load per lane from L2.  A wave
// works on 64 samples (four 16-sample tiles) per pass, so each A fragment
// loaded serves four MFMAs: 232 KiB of weight reads per 64 samples.
//
// Encoding.  Lane l of a wave evaluates the 30 + 12 sincos pairs of sample l
// of its group once and writes the sample's density input (64 halves) and
// direction encoding (27 halves and zeros) as one LDS row; lane (g, s) of
// tile t then reads its B operands back with 16-byte LDS loads.
#include "mlp_device.hpp"
#include "wave.hpp"

namespace nerf_hip {
namespace {

using namespace mlp;

constexpr uint32_t kRefDensityParams = NERF_EXT_REF_DENSITY_PARAMS;
constexpr uint32_t kRefColorParams   = NERF_EXT_REF_COLOR_PARAMS;

// Layers in consumption order: (rows out, columns in, k-blocks, row blocks,
// k-map, first fragment, offset of W in its parameter set).
enum RefMap : uint32_t { kMapIdentity = 0u, kMapHidden = 1u, kMapColorIn = 2u };
struct RefLayer {
    uint32_t n_out, n_in, kb, rb, map, frag0, w_off, network;
};
constexpr RefLayer kRefLayers[10] = {
    {128u, 64u, 2u, 8u, kMapIdentity, 0u, 0u, 0u},    {128u, 128u, 4u, 8u, kMapHidden, 16u, 8192u, 0u},  {128u, 128u, 4u, 8u, kMapHidden, 48u, 24576u, 0u},
    {128u, 128u, 4u, 8u, kMapHidden, 80u, 40960u, 0u}, {128u, 128u, 4u, 8u, kMapHidden, 112u, 57344u, 0u}, {16u, 128u, 4u, 1u, kMapHidden, 144u, 73728u, 0u},
    {128u, 48u, 2u, 8u, kMapColorIn, 148u, 0u, 1u},    {128u, 128u, 4u, 8u, kMapHidden, 164u, 6144u, 1u}, {128u, 128u, 4u, 8u, kMapHidden, 196u, 22528u, 1u},
    {16u, 128u, 4u, 1u, kMapHidden, 228u, 38912u, 1u},
};
static_assert(kRefLayers[5].w_off + 16u * 128u == kRefDensityParams, "density layout");
static_assert(kRefLayers[9].w_off + 16u * 128u == kRefColorParams, "colour layout");
constexpr uint32_t kRefFwdFragments = 232u;

// Backward products delta_in = W^T delta_out, in the order the backward
// consumes them: transposed fragments of layer `src` — rows = its input
// neurons, k = its output neurons under the hidden k-map (outputs >= n_out
// are zero).  `geo`: the colour input layer restricted to the geometry
// features, with row o = density output o (column o - 1; row 0 zero), so the
// result lands where the density output layer's deltas live.
struct RefTLayer {
    uint32_t src, rb, kb, frag0, geo;
};
constexpr RefTLayer kRefT[9] = {{9u, 8u, 1u, 232u, 0u}, {8u, 8u, 4u, 240u, 0u}, {7u, 8u, 4u, 272u, 0u}, {6u, 1u, 4u, 304u, 1u}, {5u, 8u, 1u, 308u, 0u},
                                {4u, 8u, 4u, 316u, 0u}, {3u, 8u, 4u, 348u, 0u}, {2u, 8u, 4u, 380u, 0u}, {1u, 8u, 4u, 412u, 0u}};
static_assert(kRefT[8].frag0 + 32u == kRefFragments, "fragment count");

// Rows of the neuron-major training buffers (fp16, in blocks of 32 samples:
// row r of sample s at element (s / 32 * rows + r) * 32 + s % 32): kActOff[l]
// is the input of layer l (the encoding, hidden activations, the colour
// input [geometry 15 | direction encoding 27 | 0 x 6]); kDltOff[l] the delta
// of layer l's output.  dW_l = delta_l x input_l^T over the samples.
constexpr uint32_t kActOff[10] = {0u, 64u, 192u, 320u, 448u, 576u, 704u, 752u, 880u, 1008u};
constexpr uint32_t kDltOff[10] = {0u, 128u, 256u, 384u, 512u, 640u, 656u, 784u, 912u, 1040u};
constexpr uint32_t kActRows = 1136u, kDltRows = 1056u;

// Input column of W for element j of lane group g in k-block q (-1: zero).
__device__ __forceinline__ int ref_column(uint32_t map, uint32_t q, uint32_t g, uint32_t j) {
    if (map == kMapIdentity) return (int)(32u * q + 8u * g + j);
    if (map == kMapHidden) return (int)(32u * q + (j < 4u ? 4u * g + j : 16u + 4u * g + (j - 4u)));
    if (q == 0u) {
        if (j < 4u) {
            const uint32_t o = 4u * g + j;  // raw density output o; output 0 (sigma) is not a colour input
            return o == 0u ? -1 : (int)(o - 1u);
        }
        return (int)(15u + 4u * g + (j - 4u));  // direction encoding 4g .. 4g + 3
    }
    const uint32_t e = 16u + 8u * g + j;  // direction encoding 16 .. 47 (27 used)
    return e < 27u ? (int)(15u + e) : -1;
}

// One workgroup of 64 threads per fragment.
__global__ __launch_bounds__(64) void k_ref_pack(const half_t* __restrict__ dparams, const half_t* __restrict__ cparams, half8_t* __restrict__ frags) {
    const uint32_t f = blockIdx.x, lane = threadIdx.x;
    if (f >= kRefFwdFragments) {
        uint32_t ti = 0u;
#pragma unroll
        for (uint32_t k = 1u; k < 9u; ++k)
            if (f >= kRefT[k].frag0) ti = k;
        const RefTLayer T  = kRefT[ti];
        const RefLayer L   = kRefLayers[T.src];
        const uint32_t loc = f - T.frag0, r = loc / T.kb, q = loc - r * T.kb;
        const uint32_t i = lane & 15u, g = lane >> 4;
        const half_t* W = (L.network == 0u ? dparams : cparams) + L.w_off;
        half8_t a;
#pragma unroll
        for (uint32_t j = 0; j < 8u; ++j) {
            const uint32_t o = (uint32_t)ref_column(kMapHidden, q, g, j);  // output neuron of layer src
            const uint32_t row = 16u * r + i;                               // input neuron (geo: density output)
            const bool ok = o < L.n_out && (!T.geo || (row >= 1u && row <= 15u));
            a[j] = ok ? W[o * L.n_in + (T.geo ? row - 1u : row)] : (half_t)0.0f;
        }
        frags[(uint64_t)f * 64u + lane] = a;
        return;
    }
    uint32_t li = 0u;
#pragma unroll
    for (uint32_t k = 1u; k < 10u; ++k)
        if (f >= kRefLayers[k].frag0) li = k;
    const RefLayer L   = kRefLayers[li];
    const uint32_t loc = f - L.frag0, r = loc / L.kb, q = loc - r * L.kb;
    const uint32_t i = lane & 15u, g = lane >> 4;
    const half_t* row = (L.network == 0u ? dparams : cparams) + L.w_off + (16u * r + i) * L.n_in;
    half8_t a;
#pragma unroll
    for (uint32_t j = 0; j < 8u; ++j) {
        const int c = ref_column(L.map, q, g, j);
        a[j]        = c < 0 ? (half_t)0.0f : row[c];
    }
    frags[(uint64_t)f * 64u + lane] = a;
}

// Weight fragments are read with buffer loads: one VGPR (lane * 16) and a
// scalar fragment offset per load.  With plain pointers the compiler hoists
// the 232 fragment addresses (two VGPRs each) out of the sample loop and
// spills.  Word 3 of the descriptor is the gfx9-family raw-buffer format;
// loads past num_records return zero.
struct FragSrc {
    __amdgpu_buffer_rsrc_t rsrc;
    uint32_t voff;  // lane * 16
};

__device__ __forceinline__ FragSrc frag_src(const half8_t* frags, uint32_t lane) {
    return FragSrc{__builtin_amdgcn_make_buffer_rsrc((void*)frags, (short)0, (int)(kRefFragments * 1024u), 0x00020000), lane * 16u};
}

__device__ __forceinline__ half8_t frag_load(const FragSrc& S, uint32_t f) {
    return __builtin_bit_cast(half8_t, __builtin_amdgcn_raw_buffer_load_b128(S.rsrc, S.voff, f * 1024u, 0));
}

// Where a training pass keeps a block of activations or deltas: the fp16
// neuron-major buffer (blocks of 32 samples) through a buffer descriptor;
// rows from `row0`, samples of this wave's group from s0; lane (g, s) of
// tile t owns rows 16 r + 4 g + e of sample s0 + 16 t + s.  The lane's part
// of the address (4 g rows, sample s) is one VGPR; the uniform row 16 r + e
// and block go in the scalar offset and the half block in the immediate —
// with plain pointers the compiler keeps a 64-bit address per row live and
// spills.
//
// put_quad stores a lane's four rows of one tile (rows 16 r + 4 g + e of
// sample s0 + 16 t + s) as one 8-byte store per lane: a 4 x 4 transpose
// across each quad of lanes (lanes s = 4 k + j, samples 16 t + 4 k + j)
// leaves lane j with row 16 r + 4 g + j at samples 16 t + 4 k .. + 3.  Two
// DPP swaps (lane j ^ 1, then j ^ 2), two byte permutes and two selects
// replace four 2-byte stores (a quarter of the store instructions, each a
// full wave of lane addresses for the address path).
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
// One block of a layer's rows is one contiguous run for k_ref_dw (rows at a
// stride of the sample count, 64 bytes per row and step, read back more
// slowly), and a group's stores land in two blocks.  A wave's group of 64 samples is blocks blk and blk + 1; tile t (16
// samples) is half t & 1 of block blk + t / 2.
struct RowStore {
    __amdgpu_buffer_rsrc_t rsrc;
    uint32_t vbase;  // bytes: 4 g * 64 + s16 * 2
    uint32_t tile;   // bytes of one block: rows * 64
    uint32_t row0;
    uint32_t vquad;  // bytes: (4 g + j) * 64 + 4 k * 2, s16 = 4 k + j
    uint32_t blk;    // first block of the group
    __device__ __forceinline__ uint32_t soff(uint32_t row_u, uint32_t t) const { return (row0 + row_u) * 64u + (blk + (t >> 1)) * tile; }
    __device__ __forceinline__ void put(uint32_t row_u, uint32_t t, half_t v) const {
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, v), rsrc, vbase + 32u * (t & 1u), soff(row_u, t), 0);
    }
    __device__ __forceinline__ void put_quad(uint32_t row_u, uint32_t t, half4_t h) const {
        constexpr int kSwap1 = 0xB1, kSwap2 = 0x4E;  // quad_perm [1, 0, 3, 2] and [2, 3, 0, 1]
        const uint32_t j = threadIdx.x & 3u;
        const uint32_t a = __builtin_bit_cast(uint32_t, half2_t{h[0], h[1]}), b = __builtin_bit_cast(uint32_t, half2_t{h[2], h[3]});
        const uint32_t a1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)a, kSwap1, 0xf, 0xf, false);
        const uint32_t b1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)b, kSwap1, 0xf, 0xf, false);
        // Even lanes: (own, next) of their first row; odd lanes: (previous,
        // own) of their second row.
        const uint32_t sel = (j & 1u) ? 0x03020706u : 0x05040100u;
        const uint32_t c = __builtin_amdgcn_perm(a1, a, sel), d = __builtin_amdgcn_perm(b1, b, sel);
        const uint32_t c2 = (uint32_t)__builtin_amdgcn_mov_dpp((int)c, kSwap2, 0xf, 0xf, false);
        const uint32_t d2 = (uint32_t)__builtin_amdgcn_mov_dpp((int)d, kSwap2, 0xf, 0xf, false);
        const bool first  = j < 2u;
        __builtin_amdgcn_raw_buffer_store_b64(u32x2{first ? c : d2, first ? c2 : d}, rsrc, vquad + 32u * (t & 1u), soff(row_u, t), 0);
    }
    __device__ __forceinline__ half_t get(uint32_t row_u, uint32_t t) const {
        return __builtin_bit_cast(half_t, __builtin_amdgcn_raw_buffer_load_b16(rsrc, vbase + 32u * (t & 1u), soff(row_u, t), 0));
    }
};

// The wave's index in its workgroup, in a scalar register: threadIdx.x >> 6
// is the same on every lane, but the compiler cannot tell, and a buffer
// offset derived from it that it takes for divergent is issued through a
// loop of one store per distinct value (readfirstlane + exec masking).
__device__ __forceinline__ uint32_t wave_index() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(half_t* buf, uint32_t rows, uint32_t np) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)buf, (short)0, (int)(rows * np * 2u), 0x00020000);
}

// max(x, 0) rounded to fp16: the accumulators are rounded (RNE), then the
// negative halves cleared as 16-bit integers — fp16 bit patterns order like
// signed integers (negative values, -0 included, are below +0), so a packed
// integer max with 0 gives exactly fp16(max(x, 0)) for every non-NaN x (two
// conversions and two packed maxima instead of four fp32 maxima and two
// conversions).
__device__ __forceinline__ half4_t relu_half4(const floatx4& a) {
    typedef short short4_t __attribute__((ext_vector_type(4)));
    const short4_t b = __builtin_bit_cast(short4_t, __builtin_convertvector(a, half4_t));
    return __builtin_bit_cast(half4_t, __builtin_elementwise_max(b, short4_t{0, 0, 0, 0}));
}

// Bit e of the result: h[e] > 0, for h from relu_half4 (non-negative fp16,
// so h[e] > 0 exactly when its bits are nonzero): a packed unsigned min with
// 1 leaves 0 or 1 in each half, and two shifts gather the four bits.  The
// min is written as an instruction: as a vector builtin the compiler sees
// through the bit casts to the fp16 values and emits a compare and a select
// per half instead.
__device__ __forceinline__ uint32_t pk_min_u16(uint32_t a, uint32_t b) {
    uint32_t d;
    asm("v_pk_min_u16 %0, %1, %2" : "=v"(d) : "v"(a), "v"(b));
    return d;
}
__device__ __forceinline__ uint32_t relu_bits(const half4_t& h) {
    const uint32_t q01 = pk_min_u16(__builtin_bit_cast(uint32_t, half2_t{h[0], h[1]}), 0x00010001u);
    const uint32_t q23 = pk_min_u16(__builtin_bit_cast(uint32_t, half2_t{h[2], h[3]}), 0x00010001u);
    const uint32_t x    = q01 | (q23 << 2);  // h0 at bit 0, h2 at 2, h1 at 16, h3 at 18
    return (x | (x >> 15)) & 0xFu;
}

// A layer of 128 outputs (8 row blocks) on KB k-blocks of input, four tiles;
// its fragments start at f0.  With kStore the fp16 outputs also go to st and
// their ReLU masks to mrow[4 slot + t] (LDS): bit 4 r + e = (row 16 r + 4 g +
// e of tile t > 0), the lane's 32 rows of one tile in one word.
template <uint32_t KB, bool kStore = false>
__device__ __forceinline__ void ref_hidden(const FragSrc& S, uint32_t f0, const half8_t (&in)[4][4], half8_t (&out)[4][4], const RowStore& st = RowStore{}, uint32_t* mrow = nullptr, uint32_t slot = 0u) {
    uint32_t mb[4] = {0u, 0u, 0u, 0u};
    half4_t lo[4];  // fp16 results of the even row block, joined with the odd one
    // Row block r + 1's fragments are requested before block r's MFMAs, so
    // their L2 latency overlaps the block's 4 KB MFMAs.
    half8_t nxt[KB];
#pragma unroll
    for (uint32_t q = 0; q < KB; ++q) nxt[q] = frag_load(S, f0 + q);
#pragma unroll
    for (uint32_t r = 0; r < 8u; ++r) {
        half8_t a[KB];
#pragma unroll
        for (uint32_t q = 0; q < KB; ++q) {
            a[q] = nxt[q];
            if (r + 1u < 8u) nxt[q] = frag_load(S, f0 + (r + 1u) * KB + q);
        }
        floatx4 acc[4];
#pragma unroll
        for (uint32_t t = 0; t < 4u; ++t) {
            acc[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (uint32_t q = 0; q < KB; ++q) acc[t] = mfma16x16x32(a[q], in[t][q], acc[t]);
        }
        // Each output vector is written whole (never element-wise into its
        // previous contents, which would keep those alive across the layer).
#pragma unroll
        for (uint32_t t = 0; t < 4u; ++t) {
            const half4_t h = relu_half4(acc[t]);
            if (r & 1u) out[t][r >> 1] = half8_t{lo[t][0], lo[t][1], lo[t][2], lo[t][3], h[0], h[1], h[2], h[3]};
            else lo[t] = h;
            if constexpr (kStore) {
                st.put_quad(16u * r, t, h);
                mb[t] |= relu_bits(h) << (4u * r);
            }
        }
        // One row block's weights in flight at a time: without the fence the
        // scheduler hoists the next blocks' fragment loads and spills.
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (kStore) {
#pragma unroll
        for (uint32_t t = 0; t < 4u; ++t) mrow[4u * slot + t] = mb[t];
    }
}

// The 16-output layer: raw accumulators of the four tiles.
__device__ __forceinline__ void ref_output(const FragSrc& S, uint32_t f0, const half8_t (&in)[4][4], floatx4 (&o)[4]) {
    half8_t a[4];
#pragma unroll
    for (uint32_t q = 0; q < 4u; ++q) a[q] = frag_load(S, f0 + q);
#pragma unroll
    for (uint32_t t = 0; t < 4u; ++t) {
        o[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (uint32_t q = 0; q < 4u; ++q) o[t] = mfma16x16x32(a[q], in[t][q], o[t]);
    }
}

// One backward product of a 128-input layer: delta_in = mask . (W^T
// delta_out) for the four tiles, mask = the forward ReLU mask of those 128
// rows (bits from ref_hidden), rounded to fp16 as the next product's B
// operand and stored for the weight gradients.
template <uint32_t KB>
__device__ __forceinline__ void ref_backward_layer(const FragSrc& S, uint32_t f0, const half8_t (&in)[4][4], half8_t (&out)[4][4], const uint32_t* mrow, uint32_t slot, const RowStore& dlt) {
    const uint32_t mb[4] = {mrow[4u * slot], mrow[4u * slot + 1u], mrow[4u * slot + 2u], mrow[4u * slot + 3u]};
    half4_t lo[4];
    // Row block r + 1's fragments are requested before block r's MFMAs, so
    // their L2 latency overlaps the block's 4 KB MFMAs.
    half8_t nxt[KB];
#pragma unroll
    for (uint32_t q = 0; q < KB; ++q) nxt[q] = frag_load(S, f0 + q);
#pragma unroll
    for (uint32_t r = 0; r < 8u; ++r) {
        half8_t a[KB];
#pragma unroll
        for (uint32_t q = 0; q < KB; ++q) {
            a[q] = nxt[q];
            if (r + 1u < 8u) nxt[q] = frag_load(S, f0 + (r + 1u) * KB + q);
        }
        floatx4 acc[4];
#pragma unroll
        for (uint32_t t = 0; t < 4u; ++t) {
            acc[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (uint32_t q = 0; q < KB; ++q) acc[t] = mfma16x16x32(a[q], in[t][q], acc[t]);
        }
#pragma unroll
        for (uint32_t t = 0; t < 4u; ++t) {
            // Rows whose forward output was cleared by the ReLU get a zero
            // delta: the accumulator's bits are anded with the mask bit
            // sign-extended to 32 bits (one bit-field extract each).  The
            // element is copied to a scalar first: this clang reads element 0
            // for __builtin_bit_cast of a vector element.
            floatx4 v = acc[t];
#pragma unroll
            for (uint32_t e = 0; e < 4u; ++e) {
                const float x = v[e];
                v[e]          = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, x) & (uint32_t)((int32_t)(mb[t] << (31u - (4u * r + e))) >> 31));
            }
            const half4_t h = __builtin_convertvector(v, half4_t);
            dlt.put_quad(16u * r, t, h);
            if (r & 1u) out[t][r >> 1] = half8_t{lo[t][0], lo[t][1], lo[t][2], lo[t][3], h[0], h[1], h[2], h[3]};
            else lo[t] = h;
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

__device__ __forceinline__ float softplus_ref(float x) {
    if (x > 20.0f) return x;
    if (x < -20.0f) return expf(x);
    return log1pf(expf(x));
}

// LDS row of one sample: density input [0, 64), direction encoding [64, 96)
// (27 values, then zeros); pitch 104 halves (208 bytes): the 16-byte reads of
// the 16 lanes of a lane group fall on distinct bank quads.
constexpr uint32_t kRefPitch = 104u;

// Frequency encoding of v into row[0, 3 + 6 levels) as fp16.  The level loop
// stays rolled (three sincos per iteration): unrolled, the scheduler
// interleaves all of them and the kernel spills.
// sin and cos of a frequency-encoding argument y = v 2^l (|y| < 2^10: world
// coordinates within 1.5 x 2^9, directions within 2^3).  Cody-Waite
// reduction: k = rint(2y / pi), r = y - k pi/2 with pi/2 split into three
// fp32 parts (pi/2 = C1 + C2 + C3 + 1.1e-23); C1 has 24 bits and k < 2^10, so
// the first fused step is exact and the residue r (|r| <= pi/4) carries about
// one rounding.  sin r and cos r are the Taylor polynomials to r^9 and r^10
// (truncation below 0.1 ulp on [-pi/4, pi/4]), then the quadrant k mod 4
// picks and signs them.  Every float in (0, 1024): at most 1.49 ulp from the
// correctly rounded sin and cos, and the fp16 rounding of the result differs
// from that of the correctly rounded value for 2 in 10^5 arguments (ties the
// fp32 error crosses).  The library sincosf spent about twice the
// instructions (full-range reduction and a large-argument branch); the
// encoding was a third of this kernel's vector instructions.
__device__ __forceinline__ void freq_sincos(float y, float& s_out, float& c_out) {
    constexpr float kTwoOverPi = 0x1.45f306p-1f;
    constexpr float kC1 = 0x1.921fb6p+0f, kC2 = -0x1.777a5cp-25f, kC3 = -0x1.ee59dap-50f;
    const float k = __builtin_rintf(y * kTwoOverPi);
    float r       = __builtin_fmaf(-k, kC1, y);
    r             = __builtin_fmaf(-k, kC2, r);
    r             = __builtin_fmaf(-k, kC3, r);
    const float z = r * r;
    float ps      = __builtin_fmaf(z, 0x1.71de3ap-19f, -0x1.a01a02p-13f);  // 1/9!, -1/7!
    ps            = __builtin_fmaf(z, ps, 0x1.111112p-7f);                 // 1/5!
    ps            = __builtin_fmaf(z, ps, -0x1.555556p-3f);                // -1/3!
    const float s = __builtin_fmaf(r * z, ps, r);
    float pc      = __builtin_fmaf(z, -0x1.27e4fcp-22f, 0x1.a01a02p-16f);  // -1/10!, 1/8!
    pc            = __builtin_fmaf(z, pc, -0x1.6c16c2p-10f);               // -1/6!
    pc            = __builtin_fmaf(z, pc, 0x1.555556p-5f);                 // 1/4!
    pc            = __builtin_fmaf(z, pc, -0.5f);
    const float c = __builtin_fmaf(z, pc, 1.0f);
    const int q   = (int)k;
    const float a = (q & 1) ? c : s, b = (q & 1) ? s : c;
    s_out         = (q & 2) ? -a : a;
    c_out         = ((q + 1) & 2) ? -b : b;
}

// Written as 4-byte pairs (row is 4-byte aligned): level l fills positions
// 3 + 6l .. 8 + 6l, so each level stores the previous level's last value
// with its first, then two pairs, and carries its last value on; position
// 3 + 6 levels (the first padding column) gets zero.
__device__ __forceinline__ void freq_row(const float v[3], uint32_t levels, half_t* row) {
    uint32_t* w = reinterpret_cast<uint32_t*>(row);
    auto pack   = [](half_t a, half_t b) { return __builtin_bit_cast(uint32_t, half2_t{a, b}); };
    w[0]        = pack(to_half_rne(v[0]), to_half_rne(v[1]));
    half_t carry = to_half_rne(v[2]);
    float f      = 1.0f;
#pragma unroll 1
    for (uint32_t l = 0; l < levels; ++l) {
        half_t sn[3], cs[3];
#pragma unroll
        for (uint32_t a = 0; a < 3u; ++a) {
            float s, c;
            freq_sincos(v[a] * f, s, c);  // v * 2^l is exact
            sn[a] = to_half_rne(s);
            cs[a] = to_half_rne(c);
        }
        w[1u + 3u * l] = pack(carry, sn[0]);
        w[2u + 3u * l] = pack(sn[1], sn[2]);
        w[3u + 3u * l] = pack(cs[0], cs[1]);
        carry          = cs[2];
        f *= 2.0f;
    }
    w[1u + 3u * levels] = pack(carry, (half_t)0.0f);
}

template <bool kFromSamples>
__global__ __launch_bounds__(kBlockThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_ref_field(const half8_t* __restrict__ frags, FieldInputs in, uint32_t n_cap, float4* __restrict__ out, float4* __restrict__ raw_out) {
    const uint32_t n = in.n_dev ? min(*in.n_dev, n_cap) : n_cap;
    __shared__ __align__(16) half_t rows[kBlockWaves][64 * kRefPitch];
    const uint32_t lane = threadIdx.x & 63u, g = lane >> 4, s16 = lane & 15u, wv = wave_index();
    half_t* R           = rows[wv];
    const FragSrc S     = frag_src(frags, lane);
    const uint32_t groups = (n + 63u) / 64u;
    for (uint32_t gi = blockIdx.x * kBlockWaves + wv; gi < groups; gi += gridDim.x * kBlockWaves) {
        // Encoding: lane = sample.
        float dt = 0.0f;  // the sample's interval (alpha_in_order)
        {
            const uint32_t q = min(gi * 64u + lane, n - 1u);
            float p[3], d[3];
            if constexpr (kFromSamples) {
                const uint32_t qs = in.sample_index ? in.sample_index[q] : q;
                const float2 td   = in.samples[qs];
                const uint32_t r  = sample_owner(in, q, qs);
                const float4 ro = in.rays[2ull * r], rd = in.rays[2ull * r + 1ull];
                dt = td.y;
                d[0] = rd.x;
                d[1] = rd.y;
                d[2] = rd.z;
                p[0] = ro.x + td.x * rd.x;
                p[1] = ro.y + td.x * rd.y;
                p[2] = ro.z + td.x * rd.z;
            } else {
#pragma unroll
                for (uint32_t a = 0; a < 3u; ++a) {
                    p[a] = in.positions[3ull * q + a];
                    d[a] = in.directions[3ull * q + a];
                }
            }
            half_t* row = R + lane * kRefPitch;
            freq_row(p, 10u, row);
            row[63] = (half_t)0.0f;
            freq_row(d, 4u, row + 64u);
#pragma unroll
            for (uint32_t k = 64u + 27u; k < 96u; ++k) row[k] = (half_t)0.0f;
        }
        __builtin_amdgcn_wave_barrier();  // LDS traffic of one wave completes in order
        half8_t x[4][4], y[4][4];
#pragma unroll
        for (uint32_t t = 0; t < 4u; ++t) {
            const half_t* r = R + (16u * t + s16) * kRefPitch;
            x[t][0]         = *reinterpret_cast<const half8_t*>(r + 8u * g);
            x[t][1]         = *reinterpret_cast<const half8_t*>(r + 32u + 8u * g);
            x[t][2] = x[t][3] = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
        }
        // Density network.
        ref_hidden<2>(S, kRefLayers[0].frag0, x, y);
        ref_hidden<4>(S, kRefLayers[1].frag0, y, x);
        ref_hidden<4>(S, kRefLayers[2].frag0, x, y);
        ref_hidden<4>(S, kRefLayers[3].frag0, y, x);
        ref_hidden<4>(S, kRefLayers[4].frag0, x, y);
        floatx4 dens[4];
        ref_output(S, kRefLayers[5].frag0, y, dens);
        // Colour input: raw density outputs 4g..4g+3 (fp16) and direction
        // encoding 4g..4g+3; then direction encoding 16 + 8g .. + 7.
#pragma unroll
        for (uint32_t t = 0; t < 4u; ++t) {
            const half_t* r  = R + (16u * t + s16) * kRefPitch + 64u;
            const half4_t de = *reinterpret_cast<const half4_t*>(r + 4u * g);
            x[t][0]          = half8_t{to_half_rne(dens[t][0]), to_half_rne(dens[t][1]), to_half_rne(dens[t][2]), to_half_rne(dens[t][3]), de[0], de[1], de[2], de[3]};
            x[t][1]          = g < 2u ? *reinterpret_cast<const half8_t*>(r + 16u + 8u * g) : half8_t{0, 0, 0, 0, 0, 0, 0, 0};
        }
        __builtin_amdgcn_wave_barrier();  // the rows are rewritten by the next pass
        ref_hidden<2>(S, kRefLayers[6].frag0, x, y);
        ref_hidden<4>(S, kRefLayers[7].frag0, y, x);
        ref_hidden<4>(S, kRefLayers[8].frag0, x, y);
        floatx4 col[4];
        ref_output(S, kRefLayers[9].frag0, y, col);
        // Lane group 0 holds raw outputs 0..3 of both networks; they pass
        // through LDS (the rows are free until the next group's encoding) so
        // that the activations run once per wave with lane = sample, not once
        // per tile on a quarter of the lanes.
        float4* RF = reinterpret_cast<float4*>(R);
        if (g == 0u) {
#pragma unroll
            for (uint32_t t = 0; t < 4u; ++t)
                RF[16u * t + s16] = make_float4((float)to_half_rne(dens[t][0]), (float)to_half_rne(col[t][0]), (float)to_half_rne(col[t][1]), (float)to_half_rne(col[t][2]));
        }
        __builtin_amdgcn_wave_barrier();
        const float4 rv   = RF[lane];
        const uint32_t st = gi * 64u + lane;
        if (st < n) {
            const bool in_order = kFromSamples && in.sample_index && in.alpha_in_order;
            const uint32_t dst  = (kFromSamples && in.sample_index && !in_order) ? in.sample_index[st] : st;
            const float sigma   = softplus_ref(rv.x);
            out[dst]            = make_float4(in_order ? render_alpha(sigma, dt) : sigma, 1.0f / (1.0f + expf(-rv.y)), 1.0f / (1.0f + expf(-rv.z)), 1.0f / (1.0f + expf(-rv.w)));
            if (raw_out) raw_out[dst] = rv;
        }
        __builtin_amdgcn_wave_barrier();  // the read completes before the next encoding rewrites the rows
    }
}

// MLP backward of the reference-model network for one batch (the forward is
// recomputed, :784-909 semantics with fp32 accumulation).  Per 64-sample
// group: the encoding and every layer's fp16 input go to `acts`, the fp16
// deltas of every layer's output to `dlts` (neuron-major in 32-sample
// blocks) for k_ref_dw.  Output deltas: fp16(loss_scale x d raw) for colour
// outputs 0..2; the geometry features' delta (colour input layer transposed,
// rows shifted onto density outputs 1..15) and fp16(loss_scale x d raw
// sigma) for the density outputs.  Samples past n get zero output deltas, so
// all their deltas are zero.  Register budget for two waves per SIMD: left
// to itself the compiler used 256 VGPRs and 27 AGPRs (one wave per SIMD);
// capped, it spills 77 VGPRs to scratch and the pass still runs faster
// (503 -> 476 us per 2^18 samples): with one wave nothing hides the weight
// fragment, LDS and MFMA latencies of the layer chain.
template <bool kFromSamples>
__global__ __launch_bounds__(kBlockThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_ref_backward(const half8_t* __restrict__ frags, FieldInputs in, uint32_t n_cap, const float4* __restrict__ draw, float loss_scale, half_t* __restrict__ acts,
                                                                half_t* __restrict__ dlts, uint32_t np) {
    __shared__ __align__(16) half_t rows[kBlockWaves][64 * kRefPitch];
    const uint32_t lane = threadIdx.x & 63u, g = lane >> 4, s16 = lane & 15u, wv = wave_index();
    half_t* R       = rows[wv];
    const FragSrc S = frag_src(frags, lane);
    // Samples: n_cap, or the count on the device (the trainer's) clamped to it.
    const uint32_t n      = in.n_dev ? min(*in.n_dev, n_cap) : n_cap;
    const uint32_t groups = (n + 63u) / 64u;
    const __amdgpu_buffer_rsrc_t ra = row_rsrc(acts, kActRows, np), rd = row_rsrc(dlts, kDltRows, np);
    for (uint32_t gi = blockIdx.x * kBlockWaves + wv; gi < groups; gi += gridDim.x * kBlockWaves) {
        const uint32_t s0    = gi * 64u, blk = gi * 2u;
        const uint32_t vbase = 4u * g * 64u + s16 * 2u;
        const uint32_t vquad = (4u * g + (s16 & 3u)) * 64u + (s16 & ~3u) * 2u;
        auto A = [&](uint32_t l) { return RowStore{ra, vbase, kActRows * 64u, kActOff[l], vquad, blk}; };
        auto D = [&](uint32_t l) { return RowStore{rd, vbase, kDltRows * 64u, kDltOff[l], vquad, blk}; };
        {
            const uint32_t q = min(s0 + lane, n - 1u);
            float p[3], d[3];
            if constexpr (kFromSamples) {
                const float2 td  = in.samples[q];
                const uint32_t r = in.sample_ray[q];
                const float4 ro = in.rays[2ull * r], rd = in.rays[2ull * r + 1ull];
                d[0] = rd.x;
                d[1] = rd.y;
                d[2] = rd.z;
                p[0] = ro.x + td.x * rd.x;
                p[1] = ro.y + td.x * rd.y;
                p[2] = ro.z + td.x * rd.z;
            } else {
#pragma unroll
                for (uint32_t a = 0; a < 3u; ++a) {
                    p[a] = in.positions[3ull * q + a];
                    d[a] = in.directions[3ull * q + a];
                }
            }
            half_t* row = R + lane * kRefPitch;
            freq_row(p, 10u, row);
            row[63] = (half_t)0.0f;
            freq_row(d, 4u, row + 64u);
#pragma unroll
            for (uint32_t k = 64u + 27u; k < 96u; ++k) row[k] = (half_t)0.0f;
            // Lane = sample: the encoding rows are stored one row per instruction.
            const uint32_t vs = (lane >> 5) * (kActRows * 64u) + (lane & 31u) * 2u, sb = blk * (kActRows * 64u);
            for (uint32_t k = 0; k < 64u; ++k) __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, row[k]), ra, vs, (kActOff[0] + k) * 64u + sb, 0);
            // Colour input columns 15..41: the direction encoding; 42..47: zero.
            for (uint32_t k = 15u; k < 48u; ++k) {
                const half_t v = k < 42u ? row[64u + (k - 15u)] : (half_t)0.0f;
                __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, v), ra, vs, (kActOff[6] + k) * 64u + sb, 0);
            }
        }
        __builtin_amdgcn_wave_barrier();
        half8_t x[4][4], y[4][4];
#pragma unroll
        for (uint32_t t = 0; t < 4u; ++t) {
            const half_t* r = R + (16u * t + s16) * kRefPitch;
            x[t][0]         = *reinterpret_cast<const half8_t*>(r + 8u * g);
            x[t][1]         = *reinterpret_cast<const half8_t*>(r + 32u + 8u * g);
            x[t][2] = x[t][3] = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
        }
        // The density input part of each LDS row (128 bytes) is free once x is
        // loaded: lane l keeps its 32 ReLU mask words (inputs of layers 1..5,
        // 7..9 x four tiles) in row l.
        __builtin_amdgcn_wave_barrier();
        uint32_t* M = reinterpret_cast<uint32_t*>(R + lane * kRefPitch);
        ref_hidden<2, true>(S, kRefLayers[0].frag0, x, y, A(1), M, 0u);
        ref_hidden<4, true>(S, kRefLayers[1].frag0, y, x, A(2), M, 1u);
        ref_hidden<4, true>(S, kRefLayers[2].frag0, x, y, A(3), M, 2u);
        ref_hidden<4, true>(S, kRefLayers[3].frag0, y, x, A(4), M, 3u);
        ref_hidden<4, true>(S, kRefLayers[4].frag0, x, y, A(5), M, 4u);
        floatx4 dens[4];
        ref_output(S, kRefLayers[5].frag0, y, dens);
#pragma unroll
        for (uint32_t t = 0; t < 4u; ++t) {
            const half_t* r  = R + (16u * t + s16) * kRefPitch + 64u;
            const half4_t de = *reinterpret_cast<const half4_t*>(r + 4u * g);
            const half4_t h  = half4_t{to_half_rne(dens[t][0]), to_half_rne(dens[t][1]), to_half_rne(dens[t][2]), to_half_rne(dens[t][3])};
#pragma unroll
            for (uint32_t e = 0; e < 4u; ++e)
                // Geometry = density outputs 1..15 at colour input row 4g + e - 1
                // (the uniform part e - 1 wraps to -1 for e = 0: the row sum is
                // taken modulo 2^32 and lands on 4g - 1).
                if (4u * g + e >= 1u) A(6).put(e - 1u, t, h[e]);
            x[t][0] = half8_t{h[0], h[1], h[2], h[3], de[0], de[1], de[2], de[3]};
            x[t][1] = g < 2u ? *reinterpret_cast<const half8_t*>(r + 16u + 8u * g) : half8_t{0, 0, 0, 0, 0, 0, 0, 0};
        }
        __builtin_amdgcn_wave_barrier();  // the rows are rewritten by the next pass
        ref_hidden<2, true>(S, kRefLayers[6].frag0, x, y, A(7), M, 5u);
        ref_hidden<4, true>(S, kRefLayers[7].frag0, y, x, A(8), M, 6u);
        ref_hidden<4, true>(S, kRefLayers[8].frag0, x, y, A(9), M, 7u);
        // Output deltas.  Lane group 0 holds outputs 0..3 of a sample.
        float4 dr[4];
#pragma unroll
        for (uint32_t t = 0; t < 4u; ++t) {
            const uint32_t st = s0 + 16u * t + s16;
            dr[t]             = st < n ? draw[st] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            const half4_t h   = g == 0u ? half4_t{to_half_rne(loss_scale * dr[t].y), to_half_rne(loss_scale * dr[t].z), to_half_rne(loss_scale * dr[t].w), (half_t)0.0f} : half4_t{0, 0, 0, 0};
#pragma unroll
            for (uint32_t e = 0; e < 4u; ++e) D(9).put(e, t, h[e]);
            x[t][0] = half8_t{h[0], h[1], h[2], h[3], 0, 0, 0, 0};
            x[t][1] = x[t][2] = x[t][3] = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
        }
        ref_backward_layer<1>(S, kRefT[0].frag0, x, y, M, 7u, D(8));
        ref_backward_layer<4>(S, kRefT[1].frag0, y, x, M, 6u, D(7));
        ref_backward_layer<4>(S, kRefT[2].frag0, x, y, M, 5u, D(6));
        // Geometry features -> density output deltas 1..15; output 0 = sigma.
        {
            floatx4 geo[4];
            ref_output(S, kRefT[3].frag0, y, geo);
#pragma unroll
            for (uint32_t t = 0; t < 4u; ++t) {
                half4_t h;
#pragma unroll
                for (uint32_t e = 0; e < 4u; ++e) h[e] = (g == 0u && e == 0u) ? to_half_rne(loss_scale * dr[t].x) : to_half_rne(geo[t][e]);
#pragma unroll
                for (uint32_t e = 0; e < 4u; ++e) D(5).put(e, t, h[e]);
                x[t][0] = half8_t{h[0], h[1], h[2], h[3], 0, 0, 0, 0};
                x[t][1] = x[t][2] = x[t][3] = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
            }
        }
        ref_backward_layer<1>(S, kRefT[4].frag0, x, y, M, 4u, D(4));
        ref_backward_layer<4>(S, kRefT[5].frag0, y, x, M, 3u, D(3));
        ref_backward_layer<4>(S, kRefT[6].frag0, x, y, M, 2u, D(2));
        ref_backward_layer<4>(S, kRefT[7].frag0, y, x, M, 1u, D(1));
        ref_backward_layer<4>(S, kRefT[8].frag0, x, y, M, 0u, D(0));
        __builtin_amdgcn_wave_barrier();  // the next group rewrites the rows
    }
}

// Weight gradients from the neuron-major buffers: dW_l[o][i] = sum over
// samples of delta_l[o][s] input_l[i][s], the samples on the MFMA reduction
// axis (A = delta rows, B = input rows, 32 samples per MFMA).  One workgroup
// per (layer, chunk of samples): per step of 32 samples it stages the
// layer's n_out delta rows and n_in input rows (64 bytes each, at most
// 16 KiB) in LDS once, double-buffered, and its four waves multiply their
// parts of the n_out x n_in product from there (a 128 x 128 layer: 64 x 64
// per wave, 4 x 4 blocks of 16 x 16 in registers).  With one wave per 64 x 64
// tile reading its rows from memory, every row was read once per tile row or
// column of its layer (2.2 times on average; 415 us per 2^18 samples; 361 us
// staged in LDS with rows at a stride of the sample count, 301 us with the
// rows in 32-sample blocks, where a step's rows are two contiguous runs).  Each workgroup writes its
// layer's partial for its chunk; k_ref_dw_reduce sums the chunks in order
// (deterministic; the same MFMA sequence per block as one wave per tile).
constexpr uint32_t kRefDwRows  = 256u;  // largest n_out + n_in
constexpr uint32_t kRefDwStage = kRefDwRows * 64u;  // bytes per step of 32 samples

// np is the row pitch of the buffers; with n_dev the rows hold
// ceil(min(*n_dev, np) / 64) groups (the rest is stale) and later chunks
// write zero partials.
__global__ __launch_bounds__(kBlockThreads) void k_ref_dw(const half_t* __restrict__ acts, const half_t* __restrict__ dlts, uint32_t np, uint32_t chunk, uint32_t chunks, float* __restrict__ partial,
                                                          const uint32_t* __restrict__ n_dev) {
    __shared__ __align__(16) unsigned char stage[2][kRefDwStage];
    // The wave index stays a vector value here: as a scalar (wave_index) the
    // pass took 393 us instead of 300 per 2^18 samples.
    const uint32_t lane = threadIdx.x & 63u, g = lane >> 4, i = lane & 15u, wv = threadIdx.x >> 6;
    const uint32_t l = blockIdx.x % 10u, kc = blockIdx.x / 10u;
    if (kc >= chunks) return;  // uniform per workgroup
    const RefLayer L    = kRefLayers[l];
    const uint32_t rows = L.n_out + L.n_in;  // staged rows: deltas, then inputs
    const uint32_t rb_all = L.n_out / 16u, cb_all = L.n_in / 16u;
    // This wave's blocks: rows split in halves and columns in halves (n_out
    // 128), or columns in quarters (n_out 16).
    uint32_t r0, nr, c0, nc;
    if (rb_all >= 2u) {
        nr = rb_all / 2u;
        r0 = (wv >> 1) * nr;
        const uint32_t half = (cb_all + 1u) / 2u;
        c0 = (wv & 1u) * half;
        nc = min(half, cb_all - c0);
    } else {
        nr = 1u;
        r0 = 0u;
        nc = cb_all / 4u;
        c0 = wv * nc;
    }
    const uint32_t n_used  = n_dev ? (min(*n_dev, np) + 63u) / 64u * 64u : np;
    const uint32_t k_begin = min(kc * chunk, n_used), k_end = min(n_used, kc * chunk + chunk);
    // Staging: thread t copies 16 bytes (8 samples) of row t / 4 + 64 j.
    const uint32_t srow = threadIdx.x >> 2, spart = threadIdx.x & 3u;
    // Row r of step k0 (a whole 32-sample block): the layer's delta rows, then
    // its input rows, each set one contiguous run of the block.
    auto row_ptr = [&](uint32_t r, uint32_t k0) -> const half_t* {
        return r < L.n_out ? dlts + ((uint64_t)(k0 / 32u) * kDltRows + kDltOff[l] + r) * 32u : acts + ((uint64_t)(k0 / 32u) * kActRows + kActOff[l] + r - L.n_out) * 32u;
    };
    // Two steps of loads in flight: the rows of step s + 2 are requested
    // before step s is multiplied (one step ahead left the workgroups
    // waiting on each step's loads: 385 us per 2^18 samples).
    auto fetch = [&](half8_t (&h)[4], uint32_t k0) {
#pragma unroll
        for (uint32_t j = 0; j < 4u; ++j) {
            const uint32_t r = srow + 64u * j;
            if (r < rows) h[j] = *reinterpret_cast<const half8_t*>(row_ptr(r, k0) + 8u * spart);
        }
    };
    auto put = [&](const half8_t (&h)[4], uint32_t b) {
#pragma unroll
        for (uint32_t j = 0; j < 4u; ++j) {
            const uint32_t r = srow + 64u * j;
            if (r < rows) *reinterpret_cast<half8_t*>(&stage[b][r * 64u + 16u * spart]) = h[j];
        }
    };
    floatx4 acc[4][4];
#pragma unroll
    for (uint32_t rb = 0; rb < 4u; ++rb)
#pragma unroll
        for (uint32_t cb = 0; cb < 4u; ++cb) acc[rb][cb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    // A fragment of block rb: delta row 16 (r0 + rb) + i, samples 8g..8g+7;
    // B fragment of block cb: input row 16 (c0 + cb) + i.
    auto multiply = [&](uint32_t b) {
        half8_t fa[4], fb[4];
#pragma unroll
        for (uint32_t q = 0; q < 4u; ++q) {
            fa[q] = q < nr ? *reinterpret_cast<const half8_t*>(&stage[b][(16u * (r0 + q) + i) * 64u + 16u * g]) : half8_t{0, 0, 0, 0, 0, 0, 0, 0};
            fb[q] = q < nc ? *reinterpret_cast<const half8_t*>(&stage[b][(L.n_out + 16u * (c0 + q) + i) * 64u + 16u * g]) : half8_t{0, 0, 0, 0, 0, 0, 0, 0};
        }
#pragma unroll
        for (uint32_t rb = 0; rb < 4u; ++rb)
#pragma unroll
            for (uint32_t cb = 0; cb < 4u; ++cb)
                if (rb < nr && cb < nc) acc[rb][cb] = mfma16x16x32(fa[rb], fb[cb], acc[rb][cb]);
    };
    half8_t ha[4], hb[4];
    // Step s (of `steps`) is multiplied from stage[s & 1]; its successor's rows
    // are in ha (s even) or hb (s odd) until they are put into the other buffer.
    const uint32_t steps = (k_end - k_begin) / 32u;
    if (steps > 0u) {
        fetch(ha, k_begin);
        put(ha, 0u);
    }
    if (steps > 1u) fetch(ha, k_begin + 32u);
    __syncthreads();
    for (uint32_t s = 0; s < steps; s += 2u) {  // two steps per trip: ha and hb swap roles
        if (s + 2u < steps) fetch(hb, k_begin + 32u * (s + 2u));
        multiply(0u);
        if (s + 1u < steps) put(ha, 1u);
        __syncthreads();
        if (s + 1u >= steps) break;  // uniform
        if (s + 3u < steps) fetch(ha, k_begin + 32u * (s + 3u));
        multiply(1u);
        if (s + 2u < steps) put(hb, 0u);
        __syncthreads();
    }
    // C lane (g, i): rows 4g + e of the delta block, column i of the input block.
    float* dst = partial + (uint64_t)kc * (kRefDensityParams + kRefColorParams) + (L.network == 0u ? 0u : kRefDensityParams) + L.w_off;
#pragma unroll
    for (uint32_t rb = 0; rb < 4u; ++rb)
#pragma unroll
        for (uint32_t cb = 0; cb < 4u; ++cb) {
            if (rb < nr && cb < nc) {
                const uint32_t col = 16u * (c0 + cb) + i;
#pragma unroll
                for (uint32_t e = 0; e < 4u; ++e) dst[(16u * (r0 + rb) + 4u * g + e) * L.n_in + col] = acc[rb][cb][e];
            }
        }
}

// Chunk partials summed in chunk order, one parameter per thread; the loads
// go out sixteen chunks at a time ahead of their in-order adds (a loop of
// one load and one add per chunk kept every load's latency on the chain:
// 73 -> 6 us for 64 chunks of 116,736 parameters).  With norm != NULL each workgroup
// also leaves its share of the squared gradient norm in norm[blockIdx.x]:
// the sum of squares of its finite values, or -1 minus that sum when one of
// them is not finite (the trainer's gradient statistics, backend-cuda.cu
// :1451-1476).
__global__ __launch_bounds__(256) void k_ref_dw_reduce(const float* __restrict__ partial, uint32_t chunks, float* __restrict__ ddensity, float* __restrict__ dcolor, double* __restrict__ norm) {
    constexpr uint32_t P = kRefDensityParams + kRefColorParams;
    __shared__ double wsq[4];
    __shared__ uint32_t wbad[4];
    double sq = 0.0;
    bool bad  = false;
    for (uint32_t j = blockIdx.x * 256u + threadIdx.x; j < P; j += gridDim.x * 256u) {
        float v = 0.0f;
        constexpr uint32_t kBatch = 16u;
        uint32_t c = 0;
        for (; c + kBatch <= chunks; c += kBatch) {
            float x[kBatch];
#pragma unroll
            for (uint32_t k = 0; k < kBatch; ++k) x[k] = partial[(uint64_t)(c + k) * P + j];
#pragma unroll
            for (uint32_t k = 0; k < kBatch; ++k) v += x[k];
        }
        for (; c < chunks; ++c) v += partial[(uint64_t)c * P + j];
        if (j < kRefDensityParams) ddensity[j] = v;
        else dcolor[j - kRefDensityParams] = v;
        if (isfinite(v)) sq += (double)v * (double)v;
        else bad = true;
    }
    if (!norm) return;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) sq += __shfl_xor(sq, o, 64);
    const bool wave_bad = __ballot(bad) != 0ull;
    if ((threadIdx.x & 63u) == 0u) {
        wsq[threadIdx.x >> 6]  = sq;
        wbad[threadIdx.x >> 6] = wave_bad ? 1u : 0u;
    }
    __syncthreads();
    if (threadIdx.x == 0u) {
        const double b = ((wsq[0] + wsq[1]) + wsq[2]) + wsq[3];
        norm[blockIdx.x] = (wbad[0] | wbad[1] | wbad[2] | wbad[3]) ? -1.0 - b : b;
    }
}

// Composite forward + backward with the reference's loss (:1095-1182), one
// wave per ray over 64-sample groups as in the training composite of the
// hash-grid model: field = (sigma = softplus(raw), sigmoid rgb), white
// background, ray weight w_r = 0.1 + 0.9 clamp(gt_a, 0, 1), loss
// w_r |pred - gt|^2, g = 2 w_r (pred - gt) inv_norm.  d raw sigma = dt
// (T_{i+1} c - S_i) . g sigmoid(raw), with sigmoid(raw) = 1 - e^-sigma for
// sigma = softplus(raw), taken as -expm1(-sigma) (exact for small sigma); the
// exact derivative where the reference divides by max(1 - alpha, 1e-6).
// With n_rays_dev / n_active_dev (the trainer) the ray count is
// min(*n_rays_dev, n_rays) and inv_norm = 1 / *n_active_dev (0 without
// active rays).
constexpr uint32_t kRefCompositeBatch = 8u;  // groups of 64 samples loaded together per ray

__global__ __launch_bounds__(256) void k_ref_composite_train(uint32_t n_rays_cap, const uint32_t* __restrict__ counts, const uint32_t* __restrict__ offsets, const float2* __restrict__ samples, const float4* __restrict__ field,
                                                              const float4* __restrict__ gt, float inv_norm_host, float4* __restrict__ draw, float* __restrict__ loss_sum, const uint32_t* __restrict__ n_rays_dev,
                                                              const uint32_t* __restrict__ n_active_dev) {
    __shared__ float wsum[kBlockWaves];
    const uint32_t lane = threadIdx.x & 63u, nw = gridDim.x * kBlockWaves;
    const uint32_t n_rays = n_rays_dev ? min(*n_rays_dev, n_rays_cap) : n_rays_cap;
    const uint32_t active = n_active_dev ? *n_active_dev : 0u;
    const float inv_norm  = n_active_dev ? (active ? 1.0f / (float)active : 0.0f) : inv_norm_host;
    float wave_loss     = 0.0f;
    for (uint32_t r = blockIdx.x * kBlockWaves + (threadIdx.x >> 6); r < n_rays; r += nw) {
        const uint32_t count = counts[r];
        if (count == 0u) continue;
        const uint32_t base = offsets[r];
        // kRefCompositeBatch groups of 64 samples loaded together before any
        // is composited (a ray has only its own wave to cover the loads).
        float4 fb[kRefCompositeBatch];
        float db[kRefCompositeBatch];
        auto load_batch = [&](uint32_t c0) {
#pragma unroll
            for (uint32_t b = 0; b < kRefCompositeBatch; ++b) {
                const uint32_t i = c0 + 64u * b + lane;
                const bool valid = i < count;
                fb[b]            = valid ? field[base + i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                db[b]            = valid ? fmaxf(samples[base + i].y, 0.0f) : 0.0f;
            }
        };
        float T = 1.0f, C[3] = {0.0f, 0.0f, 0.0f};
        for (uint32_t c00 = 0; c00 < count; c00 += 64u * kRefCompositeBatch) {
            load_batch(c00);
#pragma unroll
            for (uint32_t b = 0; b < kRefCompositeBatch; ++b) {
                if (c00 + 64u * b >= count) break;  // uniform
                const bool valid = c00 + 64u * b + lane < count;
                const float4 f   = fb[b];
                const float dt   = db[b];
                const float a    = valid ? -expm1f(-(f.x * dt)) : 0.0f;
                const float incl = wave::inclusive_product(1.0f - a);
                const float excl = wave::shift_up1(incl, 1.0f);
                const float w    = T * excl * a;
                C[0] += w * f.y;
                C[1] += w * f.z;
                C[2] += w * f.w;
                T *= wave::broadcast(incl, 63u);
            }
        }
        const float4 g4    = gt[r];
        const float gtv[3] = {g4.x, g4.y, g4.z};
        const float wr     = 0.1f + 0.9f * fminf(1.0f, fmaxf(0.0f, g4.w));
        float pred[3], gr[3], ray_loss = 0.0f;
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            pred[c]       = wave::sum(C[c]) + T;  // white background
            const float x = pred[c] - gtv[c];
            ray_loss += wr * x * x;
            gr[c] = 2.0f * wr * x * inv_norm;
        }
        wave_loss += ray_loss;
        T = 1.0f;
        float carry[3] = {0.0f, 0.0f, 0.0f};
        for (uint32_t c00 = 0; c00 < count; c00 += 64u * kRefCompositeBatch) {
            load_batch(c00);
#pragma unroll
            for (uint32_t b = 0; b < kRefCompositeBatch; ++b) {
                const uint32_t c0 = c00 + 64u * b;
                if (c0 >= count) break;  // uniform
                const uint32_t i  = c0 + lane;
                const bool valid  = i < count;
                const float4 f    = fb[b];
                const float dt    = db[b];
                const float a     = valid ? -expm1f(-(f.x * dt)) : 0.0f;
                const float incl  = wave::inclusive_product(1.0f - a);
                const float excl  = wave::shift_up1(incl, 1.0f);
                const float w     = T * excl * a;
                const float Tn    = T * incl;
                const float c3[3] = {f.y, f.z, f.w};
                float ds = 0.0f, dc[3];
#pragma unroll
                for (int c = 0; c < 3; ++c) {
                    const float prefix = carry[c] + wave::inclusive_sum(w * c3[c]);
                    ds += gr[c] * (Tn * c3[c] - (pred[c] - prefix));
                    dc[c]    = w * gr[c] * c3[c] * (1.0f - c3[c]);
                    carry[c] = wave::broadcast(prefix, 63u);
                }
                if (valid) draw[base + i] = make_float4(dt * ds * -expm1f(-f.x), dc[0], dc[1], dc[2]);
                T *= wave::broadcast(incl, 63u);
            }
        }
    }
    if (lane == 0u) wsum[threadIdx.x >> 6] = wave_loss;
    __syncthreads();
    if (threadIdx.x == 0u) {
        const float b = wsum[0] + wsum[1] + wsum[2] + wsum[3];
        if (b != 0.0f) atomicAdd(loss_sum, b);
    }
}

// Host-side Xavier-uniform init of backend-cuda.cu:1810-1847 on the
// reference's own shapes.
void ref_mlp_init_host(uint32_t network, float* out) {
    const uint64_t state0 = network == 0u ? nerf_math::stream_state(0x1234ull, 0x5678ull) : nerf_math::stream_state(0x9abcull, 0xdef0ull);
    uint64_t draw = 0, off = 0;
    for (const RefLayer& L : kRefLayers) {
        if (L.network != network) continue;
        const float scale    = sqrtf(6.0f / (float)(L.n_in + L.n_out));
        const uint64_t count = (uint64_t)L.n_in * L.n_out;
        for (uint64_t i = 0; i < count; ++i, ++draw) {
            const uint64_t z = nerf_math::splitmix_at(state0, draw);
            out[off + i]     = ((float)((uint32_t)(z >> 32) >> 8) * (1.0f / 16777216.0f) * 2.0f - 1.0f) * scale;
        }
        off += count;
    }
}

}  // namespace

hipError_t ref_pack_weights(const half_t* dparams, const half_t* cparams, half8_t* frags, hipStream_t stream) {
    k_ref_pack<<<kRefFragments, 64, 0, stream>>>(dparams, cparams, frags);
    return hipGetLastError();
}

hipError_t launch_ref_field(const half8_t* frags, const FieldInputs& in, uint32_t n, float4* out, float4* raw, hipStream_t stream) {
    if (n == 0u) return hipSuccess;
    const uint32_t groups = (n + 63u) / 64u;
    const uint32_t need   = (groups + kBlockWaves - 1u) / kBlockWaves;
    const uint32_t cap    = device_cu_count() * 2u;
    const uint32_t blocks = need < cap ? need : cap;
    if (in.samples) k_ref_field<true><<<blocks, kBlockThreads, 0, stream>>>(frags, in, n, out, raw);
    else k_ref_field<false><<<blocks, kBlockThreads, 0, stream>>>(frags, in, n, out, raw);
    return hipGetLastError();
}

static_assert(kActRows == kRefActRows && kDltRows == kRefDltRows, "training buffer rows");

hipError_t launch_ref_composite_train(const RefTrainLaunch& T, const uint32_t* kept, const uint32_t* offsets, const float2* samples, const float4* field, const float4* gt, float4* draw, float* loss_sum,
                                      const uint32_t* n_rays_dev, const uint32_t* n_active_dev, hipStream_t st) {
    const uint32_t waves = (T.max_rays + kBlockWaves - 1u) / kBlockWaves;
    const uint32_t cap   = device_cu_count() * 16u;
    k_ref_composite_train<<<waves < cap ? (waves ? waves : 1u) : cap, kBlockThreads, 0, st>>>(T.max_rays, kept, offsets, samples, field, gt, 0.0f, draw, loss_sum, n_rays_dev, n_active_dev);
    return hipGetLastError();
}

hipError_t launch_ref_backward_train(const RefTrainLaunch& T, const FieldInputs& in, const float4* draw, float loss_scale, float* grad, double* norm, hipStream_t st) {
    const uint32_t need = T.np / 64u / kBlockWaves + 1u, cap = device_cu_count() * 2u;
    k_ref_backward<true><<<need < cap ? need : cap, kBlockThreads, 0, st>>>(T.frags, in, T.np, draw, loss_scale, T.acts, T.dlts, T.np);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    k_ref_dw<<<10u * T.chunks, kBlockThreads, 0, st>>>(T.acts, T.dlts, T.np, kRefDwChunk, T.chunks, T.partial, in.n_dev);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    k_ref_dw_reduce<<<kRefReduceBlocks, 256, 0, st>>>(T.partial, T.chunks, grad, grad + kRefDensityParams, norm);
    return hipGetLastError();
}

}  // namespace nerf_hip

using namespace nerf_hip;

extern "C" {

NERF_API NerfStatus nerf_ext_ref_mlp_init(uint32_t network, float* params_host) {
    NERF_CHECK_ARG(network <= 1u, "nerf_ext_ref_mlp_init: network must be 0 (density) or 1 (colour)");
    NERF_CHECK_ARG(params_host, "nerf_ext_ref_mlp_init: null output");
    ref_mlp_init_host(network, params_host);
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_ref_field_forward(const uint16_t* density_params, const uint16_t* color_params, const float* positions, const float* directions, uint32_t n, float* out, float* raw, void* stream) {
    if (n == 0u) return NERF_STATUS_OK;
    NERF_CHECK_ARG(density_params && color_params && positions && directions && out, "nerf_ext_ref_field_forward: null pointer");
    hipStream_t st  = (hipStream_t)stream;
    half8_t* frags = nullptr;
    NERF_HIP_TRY(hipMallocAsync((void**)&frags, sizeof(half8_t) * 64u * kRefFragments, st));
    FieldInputs in{};
    in.positions  = positions;
    in.directions = directions;
    hipError_t e  = ref_pack_weights((const half_t*)density_params, (const half_t*)color_params, frags, st);
    if (e == hipSuccess) e = launch_ref_field(frags, in, n, (float4*)out, (float4*)raw, st);
    const hipError_t f = hipFreeAsync(frags, st);
    NERF_HIP_TRY(e);
    NERF_HIP_TRY(f);
    return NERF_STATUS_OK;
}

}  // extern "C"

namespace {
// nerf_ext_ref_backward, with the neuron-major rows in the caller's buffers
// when acts_out / dlts_out are given (else in temporary ones).
NerfStatus ref_backward(const char* who, const uint16_t* density_params, const uint16_t* color_params, const float* positions, const float* directions, const float* draw, uint32_t n, float loss_scale, float* ddensity,
                        float* dcolor, uint16_t* acts_out, uint16_t* dlts_out, void* stream) {
    if (n == 0u) return NERF_STATUS_OK;
    NERF_CHECK_ARG(density_params && color_params && positions && directions && draw && ddensity && dcolor, std::string(who) + ": null pointer");
    NERF_CHECK_ARG(n <= (1u << 20), std::string(who) + ": at most 2^20 samples per call (buffer descriptors address < 4 GiB)");
    hipStream_t st        = (hipStream_t)stream;
    const uint32_t np     = (n + 63u) / 64u * 64u;
    const uint32_t chunk  = kRefDwChunk;
    const uint32_t chunks = (np + chunk - 1u) / chunk;
    half8_t* frags = nullptr;
    half_t *acts = (half_t*)acts_out, *dlts = (half_t*)dlts_out;
    float* partial = nullptr;
    NERF_HIP_TRY(hipMallocAsync((void**)&frags, sizeof(half8_t) * 64u * kRefFragments, st));
    if (!acts_out) NERF_HIP_TRY(hipMallocAsync((void**)&acts, sizeof(half_t) * (uint64_t)kActRows * np, st));
    if (!dlts_out) NERF_HIP_TRY(hipMallocAsync((void**)&dlts, sizeof(half_t) * (uint64_t)kDltRows * np, st));
    NERF_HIP_TRY(hipMallocAsync((void**)&partial, sizeof(float) * (uint64_t)chunks * (kRefDensityParams + kRefColorParams), st));
    FieldInputs in{};
    in.positions  = positions;
    in.directions = directions;
    hipError_t e  = ref_pack_weights((const half_t*)density_params, (const half_t*)color_params, frags, st);
    if (e == hipSuccess) {
        const uint32_t need = np / 64u / kBlockWaves + 1u, cap = device_cu_count() * 2u;
        k_ref_backward<false><<<need < cap ? need : cap, kBlockThreads, 0, st>>>(frags, in, n, (const float4*)draw, loss_scale, acts, dlts, np);
        e = hipGetLastError();
    }
    if (e == hipSuccess) {
        k_ref_dw<<<10u * chunks, kBlockThreads, 0, st>>>(acts, dlts, np, chunk, chunks, partial, nullptr);
        e = hipGetLastError();
    }
    if (e == hipSuccess) {
        k_ref_dw_reduce<<<kRefReduceBlocks, 256, 0, st>>>(partial, chunks, ddensity, dcolor, nullptr);
        e = hipGetLastError();
    }
    const hipError_t f[4] = {hipFreeAsync(partial, st), dlts_out ? hipSuccess : hipFreeAsync(dlts, st), acts_out ? hipSuccess : hipFreeAsync(acts, st), hipFreeAsync(frags, st)};
    NERF_HIP_TRY(e);
    for (hipError_t x : f) NERF_HIP_TRY(x);
    return NERF_STATUS_OK;
}
}  // namespace

extern "C" {

NERF_API NerfStatus nerf_ext_ref_backward(const uint16_t* density_params, const uint16_t* color_params, const float* positions, const float* directions, const float* draw, uint32_t n, float loss_scale, float* ddensity,
                                        float* dcolor, void* stream) {
    return ref_backward("nerf_ext_ref_backward", density_params, color_params, positions, directions, draw, n, loss_scale, ddensity, dcolor, nullptr, nullptr, stream);
}

NERF_API NerfStatus nerf_ext_ref_backward_rows(const uint16_t* density_params, const uint16_t* color_params, const float* positions, const float* directions, const float* draw, uint32_t n, float loss_scale, float* ddensity,
                                             float* dcolor, uint16_t* acts, uint16_t* dlts, void* stream) {
    NERF_CHECK_ARG(n == 0u || (acts && dlts), "nerf_ext_ref_backward_rows: null row buffer");
    return ref_backward("nerf_ext_ref_backward_rows", density_params, color_params, positions, directions, draw, n, loss_scale, ddensity, dcolor, acts, dlts, stream);
}

NERF_API NerfStatus nerf_ext_ref_composite_backward(const uint32_t* counts, const uint32_t* offsets, const float* samples, const float* field, const float* gt, uint32_t n_rays, float inv_norm, float* draw, float* loss_sum,
                                                  void* stream) {
    if (n_rays == 0u) return NERF_STATUS_OK;
    NERF_CHECK_ARG(counts && offsets && samples && field && gt && draw && loss_sum, "nerf_ext_ref_composite_backward: null pointer");
    const uint32_t waves  = (n_rays + kBlockWaves - 1u) / kBlockWaves;
    const uint32_t cap    = device_cu_count() * 16u;
    k_ref_composite_train<<<waves < cap ? waves : cap, kBlockThreads, 0, (hipStream_t)stream>>>(n_rays, counts, offsets, (const float2*)samples, (const float4*)field, (const float4*)gt, inv_norm, (float4*)draw, loss_sum, nullptr,
                                                                                                nullptr);
    NERF_LAUNCH_CHECK("k_ref_composite_train");
    return NERF_STATUS_OK;
}

}  // extern "C"
