// Kernel argument blocks shared by the host library (g++) and the gfx950 kernels (hipcc).
// Every kernel takes exactly one of these structs by value; the host packs the same struct
// and hands hipModuleLaunchKernel a pointer to it. Plain C layout: u64 device addresses,
// u32 sizes, f32 scalars, so both compilers agree on offsets.
#ifndef GH_KARGS_H
#define GH_KARGS_H
#include <stdint.h>

// Device layout of a Q4_K weight [rows][nb = cols/256 blocks] (lossless 16-byte permutation of
// the GGUF bytes, same 144 B per block):
//   QS plane at 0          : chunk (row, h, u) at row*128*nb + h*64*nb + 16*u, where unit
//                            u = 4*b + g and the chunk holds qs bytes [32g+16h, 32g+16h+16) of
//                            block b (g in 0..3 is the 32-byte qs group, h in 0..1 its half).
//   HDR plane at rows*128*nb: 16 bytes per (row, b) = d, dmin, scales[12] of block b verbatim.
// Device layout of a Q6_K weight [rows][nb] (same 210 B per block):
//   QL/QH plane at 0       : chunk (row, p, u) at row*192*nb + p*64*nb + 16*u, u = 4*b + 2*s + h,
//                            p = 0: ql[64s + 16h, +16), p = 1: ql[64s + 32 + 16h, +16),
//                            p = 2: qh[32s + 16h, +16)  (s = 128-value segment, h = half).
//   SC plane at rows*192*nb: 16 bytes per (row, b) = the int8 scales[16] verbatim.
//   D plane at rows*208*nb : 2 bytes per (row, b) = d (f16).
#define GH_Q4K_QS_BYTES 128u
#define GH_Q6K_QLH_BYTES 192u

// Units of 64 k per split of a prefill GEMM's K range: whole 256-weight blocks (4 units), so
// that every split's weight stream starts on a block boundary (the producers fetch a block's
// bytes of a row together). Split z covers units [z·per, min(units, (z + 1)·per)); units is a
// multiple of 4 (in_dim a multiple of 256). Shared by the kernels and the host's split plans.
static inline
#ifdef __HIPCC__
__host__ __device__
#endif
uint32_t gh_gemm_split_units(uint32_t units, uint32_t splits) {
    return ((units / 4 + splits - 1) / splits) * 4;
}

struct GhRepackArgs {
    uint64_t src;   // GGUF block bytes
    uint64_t dst;   // device layout
    uint32_t rows;
    uint32_t nb;    // blocks per row
};

struct GhDequantArgs {
    uint64_t w;     // device layout base
    uint64_t out;   // f32 [rows][nb*256]
    uint64_t row_ptr;  // optional u32* on the device: first row (embedding token id); 0 = use row0
    uint32_t wrows; // total rows of the matrix (plane offsets)
    uint32_t nb;
    uint32_t row0;
    uint32_t rows;
    uint64_t row_list;  // optional u32[rows] on the device: row r dequantizes row_list[r]
};

// Decode GEMV epilogues (what happens to an output row's FP32 dot product).
#define GH_EPI_F16 0      // out[row] = f16(acc)                         (matmul)
#define GH_EPI_F32 1      // out[row] = acc                              (logits)
#define GH_EPI_RESID 2    // out[row] += f32(f16(acc)), out is the FP32 residual (matmul+residual_add)
#define GH_EPI_ROPE 3     // query rows (2i, 2i+1): f16, rotated at pos, x post[pos], f16 at out[row]
#define GH_EPI_CACHE 4    // f16(acc) at out[pos*rows + row] (the V cache row of this position)
#define GH_EPI_SWIGLU 5   // out[row] = f16(f16(silu(f16(gate))) * f16(up)); up weights in `aux`
#define GH_EPI_ROPE_CACHE 6  // key rows: as GH_EPI_ROPE without post-scale, at out[pos*rows+row]

// One matrix of a (possibly fused) GEMV launch. Wavefront tasks [task0, next task0) of the
// launch belong to it; each task covers R consecutive rows.
struct GhGemvSeg {
    uint64_t w;      // device layout base
    uint64_t out;    // destination base (meaning set by epi)
    uint32_t rows;   // out_dim
    uint32_t fmt;    // 12 = Q4_K, 14 = Q6_K
    uint32_t epi;    // GH_EPI_*
    uint32_t task0;  // first task index
};

// Waves per workgroup of the direct-x GEMV kernels (gh_gemv_q*_r*_d): 512-thread workgroups.
#define GH_DIRECT_WAVES 8u

struct GhGemvArgs {
    GhGemvSeg seg[3];
    uint64_t x;        // f16 activations, token-major [n][in_dim]
    uint64_t table;    // GH_EPI_ROPE: float2 (cos, sin) [positions][pairs]
    uint64_t post;     // GH_EPI_ROPE: f32 post-scale [positions] (0 = 1.0, keys)
    uint64_t pos_ptr;  // optional u32* position on the device (added to base)
    uint64_t aux;      // GH_EPI_SWIGLU: the up matrix (same shape/format as seg[0])
    uint64_t norm_w;   // nonzero: x is the FP32 residual row and the launch stages
                       // f16(x · 1/sqrt(Σx²/in_dim + eps) · norm_w) (rmsnorm_x fused)
    float eps;
    uint32_t pad2;
    uint32_t in_dim;
    uint32_t nseg;
    uint32_t n;        // tokens (> 1 only with GH_EPI_F16 / GH_EPI_F32)
    uint32_t base;     // position (GH_EPI_ROPE / GH_EPI_CACHE)
    uint32_t pairs;    // rope pairs per head (rope_dim / 2)
    uint32_t head_dim;
    uint32_t tasks;    // total tasks of the launch
    uint32_t groups;   // workgroups launched (256 threads each): read from here rather than
                       // from the dispatch packet, whose fields cost a memory round trip
};

// One matrix of a multi-matrix prefill GEMM launch (gh_gemm3_mixed_*): row tiles
// [tile0, next tile0) of the launch belong to it; its columns sit at col0 .. col0 + rows - 1 of
// the launch's FP32 partials [splits][n][Σ rows].
#define GH_GEMM_ROLE_PLAIN 0
#define GH_GEMM_ROLE_ROPE_QUERY 1  // RoPE with the query post-scale
#define GH_GEMM_ROLE_ROPE_KEY 2    // RoPE without post-scale
struct GhGemmSeg {
    uint64_t w;      // device layout weights [rows][in_dim]
    uint64_t out;    // f16 [n][rows]
    uint32_t rows;
    uint32_t fmt;    // 12 = Q4_K, 14 = Q6_K
    uint32_t tile0;
    uint32_t col0;
    uint32_t role;   // split reduce: GH_GEMM_ROLE_*
    uint32_t pad;
};

// Prefill GEMM (gemm.hip): out f16 [n][rows] (or FP32 split partials [splits][n][rows]).
#define GH_GEMM_EPI_F16 0   // out = f16(acc)
#define GH_GEMM_EPI_SILU 1  // out = silu_mul(gate, f16(acc)), gate FP16 [n][rows] in `aux`
struct GhGemmArgs {
    uint64_t x;     // f16 activations [n][in_dim]
    uint64_t w;     // device layout weights [rows][in_dim]
    uint64_t out;   // f16 [n][rows]
    uint64_t part;  // FP32 partials when splits > 1
    uint32_t in_dim;
    uint32_t rows;
    uint32_t n;
    uint32_t splits;
    uint64_t aux;     // GH_GEMM_EPI_SILU: the gate; gh_gemm_tail: the FP32 residual x [n][rows]
    uint64_t norm;    // gh_gemm_tail: FP16 RMSNorm weight [rows] (0: residual add only)
    uint64_t normed;  // gh_gemm_tail: FP16 normalized rows [n][rows]
    uint32_t epi;     // GH_GEMM_EPI_*
    float eps;        // gh_gemm_tail
    uint64_t table;   // gh_gemm_reduce_seg: float2 (cos, sin) [positions][pairs]
    uint64_t post;    // gh_gemm_reduce_seg: f32 query post-scale [positions]
    uint32_t base;    // gh_gemm_reduce_seg: position of token 0
    uint32_t head_dim;
    uint32_t pairs;   // rope_dim / 2 (pairs rotated per head)
    uint32_t nseg;    // > 0: gh_gemm3_mixed_* / gh_gemm_reduce_seg over seg[] (rows = Σ rows)
    GhGemmSeg seg[3];
};

struct GhRmsnormArgs {
    uint64_t out;   // f16 [rows][dim]
    uint64_t x;     // f32 [rows][dim]
    uint64_t w;     // f16 [dim]
    uint32_t dim;
    uint32_t rows;
    float eps;
    uint32_t pad;
};

// RoPE over `rows` packed rows of `heads` heads; row r sits at absolute position base + r (or
// base + *pos_ptr when pos_ptr != 0). table: float2 (cos, sin) [positions][pairs];
// post: f32 [positions] query post-scale (role 0) — 1.0 for keys.
struct GhRopeArgs {
    uint64_t x;       // f16 [rows][heads][head_dim], rotated in place
    uint64_t table;
    uint64_t post;    // 0 for keys
    uint64_t pos_ptr; // optional u32* position on the device
    uint32_t heads;
    uint32_t head_dim;
    uint32_t pairs;   // rope_dim / 2
    uint32_t base;
    uint32_t rows;
    uint32_t pad;
};

struct GhEltArgs {
    uint64_t out;
    uint64_t a;
    uint64_t b;
    uint32_t n;
    uint32_t pad;
};

// KV append of `vectors_k` K values (and V) at element offsets (off + pos*stride) when pos_ptr.
struct GhKvWriteArgs {
    uint64_t kc;
    uint64_t vc;
    uint64_t k;
    uint64_t v;
    uint64_t pos_ptr;    // optional u32* position; element offset = base + (*pos_ptr)*stride
    uint64_t k_off;      // element offsets into the caches
    uint64_t v_off;
    uint32_t k_count;    // elements to copy
    uint32_t v_count;
    uint32_t k_stride;   // elements per position (pos_ptr mode)
    uint32_t v_stride;
};

// Split-K flash decode: grid (splits, kv_heads, rows). Row r attends positions 0..pos_r where
// pos_r = base + r (+ *pos_ptr). Partials: m, l [rows][q_heads][splits],
// acc [rows][q_heads][splits][value_dim]; counters u32 [rows][kv_heads], zero between launches.
struct GhAttnArgs {
    uint64_t q;        // f16 [rows][q_heads][key_dim]
    uint64_t kc;       // f16 cache base [layer][context][kv_heads][key_dim]
    uint64_t vc;
    uint64_t out;      // f16 [rows][q_heads][value_dim]
    uint64_t part_m;   // f32 workspace
    uint64_t part_l;
    uint64_t part_acc;
    uint64_t pos_ptr;  // optional u32* position
    uint64_t counters; // u32 [rows][kv_heads]
    uint32_t key_dim;
    uint32_t value_dim;
    uint32_t kv_heads;
    uint32_t q_heads;
    uint32_t layer;
    uint32_t context;
    uint32_t base;
    uint32_t rows;
    uint32_t splits;   // grid.x: workgroups per (row, kv head), <= 32
    float scale;
};

// Device top-k (read_topk): gh_topk_partial keeps the `width` smallest keys of each stripe of
// `per` logits (grid = stripes); gh_topk_final merges the stripes' lists and writes the first
// k as (u32 index, f32 bits) pairs.
struct GhTopkArgs {
    uint64_t logits;   // f32 [n]
    uint64_t part;     // u64 keys [stripes][width]
    uint64_t out;      // u32 [2][k]: indices, then raw logit bits
    uint32_t n;
    uint32_t per;      // logits per stripe
    uint32_t stripes;
    uint32_t width;    // power of 2 >= k, <= 128
    uint32_t k;
};

struct GhArgmaxArgs {
    uint64_t logits;   // f32 [n]
    uint64_t part_v;   // f32 [blocks]
    uint64_t part_i;   // u32 [blocks]
    uint64_t out;      // u32 result
    uint64_t out2;     // optional second u32 destination (next token id for graph replay)
    // optional end of a replayed greedy decode step: scalars u32[0] = position, [1] = token
    // id; gh_argmax_final stores the result r in history[position], then sets token = r and
    // position + 1 (0: not a decode step)
    uint64_t step_scalars;
    uint64_t step_history;
    uint32_t n;
    uint32_t blocks;
};


#endif
