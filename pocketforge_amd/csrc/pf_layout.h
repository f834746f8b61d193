// Data layouts in HBM shared by the host runtime and the gfx950 kernels.
#pragma once
#include <stdint.h>

namespace pf {

// ---------------------------------------------------------- weight formats
enum Fmt : int32_t { FMT_Q4 = 0, FMT_Q2 = 1, FMT_Q15 = 2, FMT_Q8 = 3 };

// Int8-activation matrices (fused QKV, O, fused gate|up, down) are stored
// in tiles of 32 output rows x 256 input columns (8 blocks of 32), the
// operand layout of v_mfma_i32_32x32x32_i8: lane l = r + 32 h of a wave
// feeds weight row r, elements 16 h .. 16 h + 15 of a block.  Tile (g, c)
// (row group g, column chunk c) is at (g * K / 256 + c) * tile_bytes and
// holds the codes as 1 KiB sets (lane l's 16 bytes at l * 16) followed by
// the 32 rows' fp16 block scales (row r's eight at codes + 16 r).
//   Q4    : 4 sets; set s covers blocks 2s and 2s + 1, 8 bytes each, where
//           byte j holds element 16h + j (low nibble) and 16h + j + 8 (high).
//   Q2/Q15: 2 sets; set s covers blocks 4s .. 4s + 3, one dword each, where
//           bits 2u, 2u + 1 of byte j hold element 16h + 4u + j.
//   Q8    : 8 sets; set s is block s, 16 bytes: byte j holds element 16h + j
//           (the MFMA operand as stored, no unpacking).
// Code values: Q4 = nibble - 8, Q2 = code - 2, Q1.5 = code - 1 (code 3 is
// rejected at upload), Q8 = the signed byte.  The fused gate|up matrix
// interleaves its halves by 16 rows: group g holds gate rows 16g .. 16g + 15,
// then up rows 16g .. 16g + 15, so the SwiGLU pairs meet in one group.
constexpr int GROUP_ROWS = 32;
__host__ __device__ constexpr uint32_t code_bytes(int fmt) { return fmt == FMT_Q8 ? 32u : (fmt == FMT_Q4 ? 16u : 8u); }
__host__ __device__ constexpr uint32_t g32_code_bytes(int fmt) { return 256u * code_bytes(fmt); }
__host__ __device__ constexpr uint32_t g32_tile_bytes(int fmt) { return g32_code_bytes(fmt) + 512u; }
__host__ __device__ constexpr int code_offset(int fmt) {
    return fmt == FMT_Q8 ? 0 : (fmt == FMT_Q4 ? 8 : (fmt == FMT_Q2 ? 2 : 1));
}

// fp32-activation GEMV matrices (tied embedding / unembedding, MTP heads)
// are row-major: codes [rows][cols/32][code_bytes] in the interchange
// element order (Q4: byte j = elements 2j (low nibble), 2j+1 (high);
// Q2/Q1.5: byte j = elements 4j..4j+3 at bits 0,2,4,6; Q8: byte j =
// element j), scales separate [rows][cols/32] fp16.  Q4 and Q8 only.

// ------------------------------------------------------------- KV cache
// One (layer, head) plane holds KV_SINK_ROWS sink rows, then `ring` window
// slots (window index w lives in slot w % ring), then `pool_cap` pooled
// rows.  K and V are separate planes of int8 [rows][head_dim] with fp32 row
// scales [rows].  ring = window + pool_block + (rows of the tallest pass)
// keeps every window entry alive until it has been folded into its pooled
// row and lets a pass write its pending rows without touching visible
// entries.
constexpr uint32_t KV_SINK_ROWS = 8;
constexpr uint32_t MAX_PASS_ROWS = 8;        // decode passes (verify: n_mtp + 1 rows)
constexpr uint32_t MAX_PREFILL_ROWS = 256;   // prompt passes (int8 MFMA GEMMs)
constexpr uint32_t MAX_SEQS = 128;           // sequences of a multi-sequence engine
constexpr uint32_t MAX_ROWS = 512;           // rows of any pass (batched verify: rows x sequences)

struct KvGeom {
    uint32_t n_layers, n_heads, head_dim;
    uint32_t sink_size, window, pool_block, max_context;
    uint32_t ring, pool_cap, rows;   // rows = KV_SINK_ROWS + ring + pool_cap
    uint32_t n_seq;                  // independent sequences (planes per layer and head)
};

struct KvPlanes {
    int8_t* k;      // [sequences][layers][heads][rows][head_dim]
    int8_t* v;
    float* ks;      // [sequences][layers][heads][rows]
    float* vs;
};

// ------------------------------------------------------ pass descriptor
// A forward pass, read by the kernels from device memory so that the
// control kernels can set up the next pass without a host round trip.
// Single-sequence passes (batch == 0) forward consecutive positions
// pos0, pos0 + 1, ... of sequence seq0.  Batched passes (batch == 1) give
// each row its own sequence rseq[r] and position rpos[r]; the rows of one
// sequence are consecutive positions in consecutive rows.
struct PassDesc {
    uint32_t pos0;                 // position of row 0 (batch == 0)
    uint32_t m;                    // rows in this pass
    uint32_t batch;
    uint32_t seq0;                 // sequence of every row (batch == 0)
    int32_t tok[MAX_ROWS];
    uint32_t rpos[MAX_ROWS];       // batch == 1
    uint32_t rseq[MAX_ROWS];
};

// Decode-loop state kept on the device.
struct DecodeState {
    uint32_t pos;          // positions stored (committed) so far
    int32_t cur;           // current token (last pushed)
    uint32_t n_tokens;     // tokens in the output buffer (prompt included)
    uint32_t n_gen;        // generated tokens
    uint64_t draw;         // stochastic draws consumed
    uint32_t accepted;     // total accepted drafts
    uint32_t rejected;     // total pushed correctives
    uint32_t have_row4;    // pass B row 4 already holds F(cur) at position pos
    uint32_t round_word;   // last round: accepted | pushed << 8
    int32_t draft[8];      // drafts of the current round
    int32_t row_argmax[8]; // greedy argmax of each pass-B row
    uint32_t round_acc;    // accepted drafts in the current round
    uint32_t n_mtp;        // drafts per MTP round (single-sequence engine)
    uint32_t seg_k0;       // draft index checked by row 0 of the current verify segment
    uint32_t more;         // the segment accepted every row it checked, drafts remain
    uint32_t blocks_done;  // finished blocks of the running k_sample_round / k_verify_accept (0 between launches)
};

struct SamplingCfg {
    float temperature;
    float top_p;
    uint32_t top_k;
    int32_t greedy;
};

}  // namespace pf
